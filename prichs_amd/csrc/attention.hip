// attention.hip -- causal GQA self-attention forward (flash-style) on CDNA4
// MFMA, for the PrichsBlock attention sub-layer.
//
// Semantics: crates/prichs-model/src/attention.rs:94-149 -- per head h with
// kv head h / (Hq / Hkv): scores = (q . k) * scale over j <= i, softmax over
// the causal row, out = sum_j p_j v_j.  The T x T score matrix is never
// materialised: each workgroup streams 64-row K/V blocks through LDS and
// keeps an online softmax per query row: a reference max m, raised only when
// a block's max passes it by more than 2^8 in p (so the output is rescaled a
// few times per row), and the row sum l = sum p, accumulated by MFMA as P
// times a ones fragment next to O += P V.
//
// Layout per workgroup: 4 wave64s, each owning 32 query rows (two 16-row
// MFMA blocks) of one query head.  With HPW heads per workgroup the 4 waves
// are HPW heads of one kv group x (4 / HPW) row blocks, so the workgroup
// covers 128 / HPW queries and every K/V tile it stages in LDS serves HPW
// query heads (HPW = 4 at 12 Q / 3 KV heads: the whole group shares a tile).
//   S^T = K Q^T     v_mfma_f32_16x16x32_bf16(K frag, Q frag): the lane owning
//                   query column q = lane % 16 holds the scores of kv rows
//                   4*(lane/16) + r of every 16-row kv block;
//   O^T += V^T P^T  v_mfma_f32_16x16x32_bf16(V^T frag, P frag): P (bf16) is
//                   taken straight from the softmax registers -- the MFMA's
//                   k index runs over kv rows {4g..4g+3, 16+4g..16+4g+3} of
//                   each 32-row step (g = lane / 16), and the V^T fragment
//                   reads the same kv rows -- so no lane exchange is needed,
//                   and the lane that owns query q also owns its output row.
// K and V go straight from global memory to LDS (global_load_lds, no VGPR
// round trip) into two stage buffers, so the next block's tiles stream in
// while this block is computed.  Both tiles are row-major [64 kv][128 d] with
// their 16-byte chunks XOR-swizzled per row (the DMA lane for LDS slot s of
// row r fetches logical chunk s ^ key(r)): K fragments are plain 16-byte
// reads, and the V^T fragments of the P.V product come from the transposing
// LDS read ds_read_b64_tr_b16 -- within each 16-lane group it hands lane i
// element j = M[4j + i/4][i % 4] of the group's 16 x 4 loaded elements, so
// lanes reading rows r0 + m/4, columns 4 (m % 4).. of a 16-column block give
// lane i that column's 4 consecutive kv values.
#include "common.hpp"

#include <type_traits>
#include <utility>

namespace prichs {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kHd = 128;      // head dim supported by this kernel
constexpr int kBKV = 64;      // kv rows per block
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kTileElems = kBKV * kHd;                   // one K or V tile [64][128]
constexpr int kStageElems = 2 * kTileElems;              // K then V
constexpr size_t kLdsBytes = 2 * (size_t)kStageElems * sizeof(bf16_t);  // two stages
constexpr float kLazy = 8.0f;  // log2 headroom of the lazily raised softmax max

__device__ __forceinline__ f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Chunk keys: K fragment reads (16 kv rows, one chunk) and V transposing
// reads (4 rows x 2 chunks per 16-lane group) both land on distinct banks.
__device__ __forceinline__ int k_key(int kv) { return kv & 15; }
__device__ __forceinline__ int v_key(int kv) { return (2 * kv) & 15; }
// Element offset of (kv row, logical 16-byte chunk c) in a K / V tile.
__device__ __forceinline__ int k_off(int kv, int c) { return kv * kHd + ((c ^ k_key(kv)) << 3); }
__device__ __forceinline__ int v_off(int kv, int c) { return kv * kHd + ((c ^ v_key(kv)) << 3); }

// Buffer resource over `bytes` bytes from `base` (raw: stride 0, gfx9 word 3).
// Loads at offsets at or past `bytes` return zeros instead of reading memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                           0x00020000);
}
// 16 bytes per lane from buffer offset voff straight into LDS at lds_dst +
// 16 * lane (lds_dst wave-uniform).
__device__ __forceinline__ void dma_16b(__amdgpu_buffer_rsrc_t r, uint32_t voff, bf16_t *lds_dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      r, (__attribute__((address_space(3))) void *)lds_dst, 16, voff, 0, 0, 0);
}
// ds_read_b64_tr_b16 as inline asm: the builtin form makes the compiler wait
// for every DMA in flight (it cannot tell the read from the DMA's target).
// OFF is the instruction's immediate byte offset.  The result is pending
// until lds_wait_tied() below, which takes the registers as operands so no
// use can be scheduled before the wait.
template <int OFF>
__device__ __forceinline__ u32x2 ds_read_tr16(uint32_t lds_byte_addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset is 16 bits");
  u32x2 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(lds_byte_addr), "n"(OFF));
  return r;
}
__device__ __forceinline__ void lds_wait_tied(u32x2 &a, u32x2 &b, u32x2 &c, u32x2 &d, u32x2 &e,
                                              u32x2 &f, u32x2 &g, u32x2 &h) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(a), "+v"(b), "+v"(c), "+v"(d), "+v"(e), "+v"(f), "+v"(g), "+v"(h)
               :
               : "memory");
}

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) { return pack_bf16x2(a, b); }

// Max over lanes l, l ^ 16, l ^ 32, l ^ 48 (the four 16-lane groups
// sharing a query column): v_permlane16_swap exchanges odd and even 16-lane
// rows, v_permlane32_swap the two wave halves.
// The maxima are IEEE 754-2019 maximum (v_maximum3_f32 on gfx950: NaN
// propagates, so no operand needs the canonicalising pass that fmaxf's
// maxNum semantics put before each raw MFMA result).
__device__ __forceinline__ float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float max_across_groups(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  x = vmax(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const uint32_t w = __float_as_uint(x);
  const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
  return vmax(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
template <bool B> using bool_c = std::integral_constant<bool, B>;
template <int I> using int_c = std::integral_constant<int, I>;
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, I...>) {
  (f(int_c<I>{}), ...);
}
// f(int_c<0>), ..., f(int_c<N - 1>): loop indices usable as template arguments.
template <int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

constexpr uint32_t kTileBytes = kTileElems * sizeof(bf16_t);
constexpr uint32_t kStageBytes = kStageElems * sizeof(bf16_t);

// q/k/v/o: row r of sequence b is row b*S + r; head h of q/o starts at column
// h*128, kv head j of k/v at column j*128 (leading dimensions ldq/ldk/ldv/ldo;
// 64 rows of k or v span less than 4 GiB).
// RoPE of one Q fragment (8 consecutive head dims 8 c .. 8 c + 7, 4 pairs)
// with the cos / sin of its pairs: the reference's rotation with each
// product and each sum rounded (crates/prichs-core/src/backward.rs:175-184),
// then bf16 -- the same operations and rounding as rope_kernel, so the result
// is the bf16 value that kernel would have stored.
__device__ __forceinline__ bf16x8 rope_frag(bf16x8 f, float4 c4, float4 s4) {
#pragma clang fp contract(off)
  u32x4 u = __builtin_bit_cast(u32x4, f);
  const float c[4] = {c4.x, c4.y, c4.z, c4.w}, sn[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float q0 = __uint_as_float(u[j] << 16), q1 = __uint_as_float(u[j] & 0xffff0000u);
    const float a0 = q0 * c[j], b0 = q1 * sn[j];
    const float a1 = q0 * sn[j], b1 = q1 * c[j];
    u[j] = pack_bf16(a0 - b0, a1 + b1);
  }
  return __builtin_bit_cast(bf16x8, u);
}

template <int HPW>
__global__ __launch_bounds__(kThreads, 2) void attn_fwd_kernel(
    const bf16_t *__restrict__ q, int ldq, const bf16_t *__restrict__ k, int ldk,
    const bf16_t *__restrict__ v, int ldv, bf16_t *__restrict__ o, int ldo, int S, int Hq,
    int group, float scale_log2, const float *__restrict__ rcos, const float *__restrict__ rsin,
    int pos_offset) {
  static_assert(kWaves % HPW == 0, "whole row blocks per head");
  constexpr int kRowsWg = 32 * kWaves / HPW;  // query rows per workgroup
  extern __shared__ __attribute__((aligned(16))) bf16_t lds[];

  // Grid (head set, sequence, query block): blocks are dispatched x-fastest,
  // so every head set's longest causal rows (the last query block) go first.
  const int n_qb = (S + kRowsWg - 1) / kRowsWg;
  const int sets = group / HPW;  // head sets per kv group
  const int kvh = blockIdx.x / sets;
  const int b = blockIdx.y;
  const int qb = n_qb - 1 - (int)blockIdx.z;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = kvh * group + (blockIdx.x - kvh * sets) * HPW + wave % HPW;
  const int g = lane >> 4;    // 0..3
  const int l16 = lane & 15;  // 0..15

  const size_t seq0 = (size_t)b * S;
  const bf16_t *kbase = k + seq0 * ldk + (size_t)kvh * kHd;
  const bf16_t *vbase = v + seq0 * ldv + (size_t)kvh * kHd;

  // Query rows of this wave: q0 + 16*nb + l16 (nb = 0, 1).
  const int q0 = qb * kRowsWg + (wave / HPW) * 32;

  // Q fragments (B operand of S^T = K Q^T): lane holds Q[q][32kk + 8g .. +8].
  bf16x8 qf[2][4];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    int qr = q0 + 16 * nb + l16;
    qr = qr < S ? qr : S - 1;
    const bf16_t *qrow = q + (seq0 + qr) * ldq + (size_t)h * kHd + 8 * g;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) qf[nb][kk] = *reinterpret_cast<const bf16x8 *>(qrow + 32 * kk);
    if (rcos != nullptr) {
      // q as projected: rotate it here (the fragment's pairs are 16 kk + 4 g ..).
      const size_t cbase = (size_t)(qr + pos_offset) * (kHd / 2) + 4 * g;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        qf[nb][kk] = rope_frag(qf[nb][kk], *reinterpret_cast<const float4 *>(rcos + cbase + 16 * kk),
                               *reinterpret_cast<const float4 *>(rsin + cbase + 16 * kk));
    }
  }

  f32x4 oacc[8][2];  // O^T blocks: d block jd, query block nb
#pragma unroll
  for (int jd = 0; jd < 8; ++jd)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) oacc[jd][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  // Reference max (log2 units) of row q: p = exp2(s - m_ref).  It is only
  // raised when a block's max exceeds it by more than kLazy, so p <= 2^kLazy
  // and the output rows are rescaled a few times per row, not per block.
  float m_ref[2] = {-INFINITY, -INFINITY};
  // Row sums of P, accumulated by MFMA against a ones fragment (every element
  // of lsum[nb] holds the sum of query row q0 + 16 nb + lane % 16).
  f32x4 lsum[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
  const bf16x8 ones = __builtin_bit_cast(bf16x8, u32x4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u,
                                                        0x3f803f80u});

  // kv blocks up to the last query row of the workgroup (causal).
  const int q_last = min(S, (qb + 1) * kRowsWg) - 1;
  const int n_kvb = q_last / kBKV + 1;

  // Loop-invariant LDS byte addresses of this lane's fragment reads within a
  // stage; rows 16c (K) and 32 ks2 / +16 (V) on share the chunk key and
  // become the instructions' immediate offsets, the stage a register add.
  //   K fragment: kv row l16 (+16c), logical chunk 4kk + g.
  //   V^T read:   kv row 4g + l16/4 (+32 ks2, +16), column 16 jd + 4 (l16 % 4).
  uint32_t k_addr[4], v_addr[8];
  const uint32_t lds_base =
      (uint32_t)(size_t)(const __attribute__((address_space(3))) bf16_t *)lds;
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) k_addr[kk] = 2u * (uint32_t)k_off(l16, 4 * kk + g);
#pragma unroll
  for (int jd = 0; jd < 8; ++jd) {
    const int col = 16 * jd + 4 * (l16 & 3);
    v_addr[jd] = lds_base + 2u * (uint32_t)(v_off(4 * g + (l16 >> 2), col >> 3) + (col & 7));
  }
  // Loop-invariant byte offsets of this lane's DMA sources within a 64-row
  // block: wave w moves rows 16 w .. 16 w + 15 of each tile, 4 rows
  // (1 KiB) per instruction, and the lane for LDS slot (row, s) fetches
  // logical chunk s ^ key(row).
  uint32_t dk[4], dv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 16 * wave + 4 * i + g;
    dk[i] = 2u * ((uint32_t)row * (uint32_t)ldk + 8u * (uint32_t)(l16 ^ k_key(row)));
    dv[i] = 2u * ((uint32_t)row * (uint32_t)ldv + 8u * (uint32_t)(l16 ^ v_key(row)));
  }

  // Block kb's K tile lives in stage buffer kb & 1 of K, its V tile in stage
  // buffer kb & 1 of V.  K runs one block ahead of V: iteration kb computes
  // S for block kb + 1 (MFMA) while the softmax of block kb (VALU) and then
  // its P.V product run, so the matrix and vector pipes overlap within a wave.
  // The buffer resources end after the sequence's last row, so rows past it
  // (last block only) load as zeros; their scores are masked.
  auto issue_tile = [&](int kb, const bf16_t *src, int ld, const uint32_t (&off)[4],
                        int tile) {
    bf16_t *dst = lds + (kb & 1) * kStageElems + tile * kTileElems;
    const uint64_t bytes = (uint64_t)(S - 1 - kb * kBKV) * 2 * (uint64_t)ld + 2 * kHd;
    const __amdgpu_buffer_rsrc_t r = buffer_rsrc(
        src + (size_t)kb * kBKV * ld, bytes > 0xffffffffull ? 0xffffffffu : (uint32_t)bytes);
#pragma unroll
    for (int i = 0; i < 4; ++i) dma_16b(r, off[i], dst + (16 * wave + 4 * i) * kHd);
  };
  auto issue_k = [&](int kb) { issue_tile(kb, kbase, ldk, dk, 0); };
  auto issue_v = [&](int kb) { issue_tile(kb, vbase, ldv, dv, 1); };
  // Every wave's DMAs issued so far have landed (each wave waits for its own,
  // the barrier for the others'), and every wave is past the reads before it.
  // s_waitcnt vmcnt(0) (gfx9 encoding: vmcnt[3:0] | expcnt 7 << 4 |
  // lgkmcnt 15 << 8 | vmcnt[5:4] << 14).
  auto sync_tiles = [&]() {
    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
    __syncthreads();
  };

  // S^T = K Q^T of block kb: 4 kv blocks x 2 query blocks; sacc[c][nb][r] =
  // raw score of (query q0 + 16nb + l16, kv 64 kb + 16c + 4g + r).
  auto compute_s = [&](int kb, f32x4 (&sacc)[4][2]) {
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) sacc[c][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
    const char *kbytes = reinterpret_cast<const char *>(lds) + (uint32_t)(kb & 1) * kStageBytes;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      bf16x8 kf[4];
#pragma unroll
      for (int c = 0; c < 4; ++c)
        kf[c] = *reinterpret_cast<const bf16x8 *>(kbytes + 16 * kHd * 2 * c + k_addr[kk]);
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) sacc[c][nb] = mfma_bf16(kf[c], qf[nb][kk], sacc[c][nb]);
    }
  };

  // Iteration kb: S of block kb + 1 into snext (past the last block the
  // stale tile it reads gives a result nobody uses), then the softmax and
  // P.V of block kb from scur.  MASKED applies the causal / length mask
  // (blocks reaching past this wave's first query row or the sequence end).
  auto run_iter = [&](int kb, auto masked_c, f32x4 (&scur)[4][2], f32x4 (&snext)[4][2]) {
    constexpr bool kMasked = decltype(masked_c)::value;
    const int kv0 = kb * kBKV;
    // K of block kb + 1 and V of block kb have landed; the buffers of K kb
    // and V kb - 1 are free for K kb + 2 and V kb + 1.
    sync_tiles();
    if (kb + 2 < n_kvb) issue_k(kb + 2);
    if (kb + 1 < n_kvb) issue_v(kb + 1);

    compute_s(kb + 1, snext);

    // Online softmax.  The block max is taken on raw scores (the scale is
    // positive, and rounding is monotone, so max(fl(s * c)) = fl(max(s) * c))
    // and p = exp2(s * scale_log2 - m_ref) is one fma per score.
    u32x4 pf[2][2];  // P fragments: [nb][32-row kv step]
    float alpha[2];
    bool raise[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      if constexpr (kMasked) {
        // Valid iff kv <= query row and kv < S, i.e. 16c + r <= lim.
        const int lim = min(q0 + 16 * nb + l16, S - 1) - kv0 - 4 * g;
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (16 * c + r > lim) scur[c][nb][r] = -INFINITY;
      }
      float mloc = -INFINITY;
#pragma unroll
      for (int c = 0; c < 4; ++c)
        mloc = vmax(vmax(vmax(mloc, scur[c][nb][0]), scur[c][nb][1]),
                    vmax(scur[c][nb][2], scur[c][nb][3]));
      mloc = max_across_groups(mloc);
      const float m_blk = mloc * scale_log2;
      // -inf + kLazy stays -inf: a row's first valid score always raises it.
      raise[nb] = m_blk > m_ref[nb] + kLazy;
      const float m_new = raise[nb] ? m_blk : m_ref[nb];
      alpha[nb] = raise[nb] ? fast_exp2(m_ref[nb] - m_new) : 1.0f;
      m_ref[nb] = m_new;
      float m_use = m_new;
      // Rows with no valid score yet keep m = -inf; exp2(-inf - -inf) would
      // be NaN.  Only a masked block can leave a row without one.
      if constexpr (kMasked) m_use = m_new == -INFINITY ? 0.f : m_new;
      const float neg_m = -m_use;
#pragma unroll
      for (int ks2 = 0; ks2 < 2; ++ks2) {
        // k slots 0..3: kv block 2 ks2 (rows 4g + r); slots 4..7: block 2 ks2 + 1.
        float p[8];
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            p[4 * h2 + r] = fast_exp2(fmaf(scur[2 * ks2 + h2][nb][r], scale_log2, neg_m));
        pf[nb][ks2] = u32x4{pack_bf16(p[0], p[1]), pack_bf16(p[2], p[3]), pack_bf16(p[4], p[5]),
                            pack_bf16(p[6], p[7])};
      }
    }
    // Pin the P fragments here: otherwise the compiler sinks the exp work
    // past the branch below, out of reach of the S MFMAs it should overlap.
    asm volatile("" ::"v"(pf[0][0]), "v"(pf[0][1]), "v"(pf[1][0]), "v"(pf[1][1]));
    // Rescale the output rows where the reference max was raised (rare).
    if (__any(raise[0] || raise[1])) {
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
        for (int jd = 0; jd < 8; ++jd) oacc[jd][nb] = oacc[jd][nb] * alpha[nb];
        lsum[nb] = lsum[nb] * alpha[nb];
      }
    }

    // O^T += V^T P^T: d blocks jd, 32-row kv steps ks2.  Lane m of each
    // 16-lane group reads row 32 ks2 + 4g + m/4 (and 16 rows on for the
    // upper half), columns 16 jd + 4 (m % 4) .. + 3; four d blocks per batch
    // of transposing reads.
    const uint32_t v_stage = (uint32_t)(kb & 1) * kStageBytes;
    static_for<2>([&](auto ks2_c) {
      constexpr int ks2 = decltype(ks2_c)::value;
      constexpr int kLo = (int)kTileBytes + 2 * 32 * ks2 * kHd;  // rows 32 ks2 + ...
      constexpr int kHi = kLo + 2 * 16 * kHd;                    // rows 32 ks2 + 16 + ...
#pragma unroll
      for (int j0 = 0; j0 < 8; j0 += 4) {
        u32x2 lo[4], hi[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const uint32_t a = v_addr[j0 + t] + v_stage;
          lo[t] = ds_read_tr16<kLo>(a);
          hi[t] = ds_read_tr16<kHi>(a);
        }
        lds_wait_tied(lo[0], hi[0], lo[1], hi[1], lo[2], hi[2], lo[3], hi[3]);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const bf16x8 vf = __builtin_bit_cast(bf16x8, u32x4{lo[t][0], lo[t][1], hi[t][0], hi[t][1]});
#pragma unroll
          for (int nb = 0; nb < 2; ++nb)
            oacc[j0 + t][nb] =
                mfma_bf16(vf, __builtin_bit_cast(bf16x8, pf[nb][ks2]), oacc[j0 + t][nb]);
        }
      }
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
        lsum[nb] = mfma_bf16(ones, __builtin_bit_cast(bf16x8, pf[nb][ks2]), lsum[nb]);
    });
  };

  // Blocks whose kv rows all lie at or before this wave's first query row
  // and inside the sequence run unmasked (two per loop trip, so the score
  // registers swap roles without copies); the rest (the diagonal and the
  // ragged tail) run masked.
  const int n_full = min(min(q0 + 1, S) / kBKV, n_kvb);
  f32x4 sa[4][2], sb[4][2];
  issue_k(0);
  sync_tiles();
  issue_v(0);
  if (n_kvb > 1) issue_k(1);
  compute_s(0, sa);
  int kb = 0;
  for (; kb + 2 <= n_full; kb += 2) {
    run_iter(kb, bool_c<false>{}, sa, sb);
    run_iter(kb + 1, bool_c<false>{}, sb, sa);
  }
  auto take_next = [&]() {
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) sa[c][nb] = sb[c][nb];
  };
  if (kb < n_full) {
    run_iter(kb, bool_c<false>{}, sa, sb);
    take_next();
    ++kb;
  }
  for (; kb < n_kvb; ++kb) {
    run_iter(kb, bool_c<true>{}, sa, sb);
    take_next();
  }

  // Normalise by the row sum and store: lane holds O[q][16 jd + 4g + r].
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const float inv = 1.0f / fmaxf(lsum[nb][0], 1e-30f);
    const int qrow = q0 + 16 * nb + l16;
    if (qrow < S) {
      bf16_t *orow = o + (seq0 + qrow) * ldo + (size_t)h * kHd + 4 * g;
#pragma unroll
      for (int jd = 0; jd < 8; ++jd) {
        const f32x4 a = oacc[jd][nb];
        *reinterpret_cast<u32x2 *>(orow + 16 * jd) =
            u32x2{pack_bf16(a[0] * inv, a[1] * inv), pack_bf16(a[2] * inv, a[3] * inv)};
      }
    }
  }
}

}  // namespace
}  // namespace prichs

using namespace prichs;

namespace prichs {
int attention_forward_impl(const void *q, size_t ldq, const void *k, size_t ldk, const void *v,
                           size_t ldv, void *o, size_t ldo, size_t batch, size_t seq_len,
                           size_t n_heads, size_t n_kv_heads, size_t head_dim, int dtype,
                           const float *rope_cos, const float *rope_sin, size_t cache_rows,
                           size_t pos_offset, void *stream) {
  PRICHS_REQUIRE(dtype == PRICHS_DTYPE_BF16, "attention: only bf16 is supported (dtype=%d)", dtype);
  if (head_dim != (size_t)kHd)
    return fail(PRICHS_ERR_UNSUPPORTED, "attention: head_dim=%zu (only %d is supported)",
                head_dim, kHd);
  PRICHS_REQUIRE(n_heads >= 1 && n_kv_heads >= 1 && n_heads % n_kv_heads == 0,
                 "attention: n_heads=%zu must be a positive multiple of n_kv_heads=%zu",
                 n_heads, n_kv_heads);
  PRICHS_REQUIRE(ldq >= n_heads * head_dim && ldo >= n_heads * head_dim &&
                     ldk >= n_kv_heads * head_dim && ldv >= n_kv_heads * head_dim,
                 "attention: leading dimensions too small");
  PRICHS_REQUIRE(ldq % 8 == 0 && ldk % 8 == 0 && ldv % 8 == 0 && ldo % 8 == 0,
                 "attention: leading dimensions must be multiples of 8 elements");
  PRICHS_REQUIRE(batch * seq_len <= (size_t)INT32_MAX && n_heads <= 65535 && batch <= 65535 &&
                     ldq <= (size_t)INT32_MAX && ldo <= (size_t)INT32_MAX,
                 "attention: shape too large");
  // The kernel addresses a 64-row K/V block with 32-bit byte offsets.
  PRICHS_REQUIRE(ldk < ((size_t)1 << 25) && ldv < ((size_t)1 << 25),
                 "attention: ldk / ldv must be below 2^25 elements");
  if (batch == 0 || seq_len == 0) return PRICHS_OK;
  PRICHS_REQUIRE(rope_cos == nullptr || (rope_sin != nullptr && seq_len + pos_offset <= cache_rows &&
                                         pos_offset <= (size_t)INT32_MAX),
                 "attention: rope cache of %zu rows does not cover positions %zu + %zu",
                 cache_rows, pos_offset, seq_len);
  PRICHS_REQUIRE(q && k && v && o, "attention: null pointer argument");
  const uintptr_t al = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                       reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(o);
  PRICHS_REQUIRE(al % 16 == 0, "attention: q/k/v/o must be 16-byte aligned");
  const int group = (int)(n_heads / n_kv_heads);
  // Heads per workgroup: the largest of 4, 2, 1 dividing the GQA group.
  const int hpw = group % 4 == 0 ? 4 : group % 2 == 0 ? 2 : 1;
  const int rows_wg = 32 * kWaves / hpw;
  const int n_qb = (int)cdiv(seq_len, (size_t)rows_wg);
  const float scale_log2 = (1.0f / sqrtf((float)head_dim)) * 1.4426950408889634f;
  PRICHS_REQUIRE(n_qb <= 65535, "attention: seq_len too large");
  const dim3 grid((unsigned)(n_heads / hpw), (unsigned)batch, (unsigned)n_qb);
  auto kern = hpw == 4 ? attn_fwd_kernel<4> : hpw == 2 ? attn_fwd_kernel<2> : attn_fwd_kernel<1>;
  hipLaunchKernelGGL(kern, grid, dim3(kThreads), kLdsBytes, as_stream(stream),
                     static_cast<const bf16_t *>(q), (int)ldq, static_cast<const bf16_t *>(k),
                     (int)ldk, static_cast<const bf16_t *>(v), (int)ldv,
                     static_cast<bf16_t *>(o), (int)ldo, (int)seq_len, (int)n_heads, group,
                     scale_log2, rope_cos, rope_sin, (int)pos_offset);
  PRICHS_LAUNCH_CHECK("attention launch");
  return PRICHS_OK;
}
}  // namespace prichs

extern "C" int prichs_attention_forward(const void *q, size_t ldq, const void *k, size_t ldk,
                                        const void *v, size_t ldv, void *o, size_t ldo,
                                        size_t batch, size_t seq_len, size_t n_heads,
                                        size_t n_kv_heads, size_t head_dim, int dtype,
                                        void *stream) {
  return attention_forward_impl(q, ldq, k, ldk, v, ldv, o, ldo, batch, seq_len, n_heads,
                                n_kv_heads, head_dim, dtype, nullptr, nullptr, 0, 0, stream);
}

extern "C" int prichs_attention_forward_rope_q(const void *q, size_t ldq, const void *k,
                                               size_t ldk, const void *v, size_t ldv, void *o,
                                               size_t ldo, size_t batch, size_t seq_len,
                                               size_t n_heads, size_t n_kv_heads,
                                               size_t head_dim, int dtype, const float *rope_cos,
                                               const float *rope_sin, size_t cache_rows,
                                               size_t pos_offset, void *stream) {
  PRICHS_REQUIRE(rope_cos && rope_sin, "attention_rope_q: null RoPE table");
  return attention_forward_impl(q, ldq, k, ldk, v, ldv, o, ldo, batch, seq_len, n_heads,
                                n_kv_heads, head_dim, dtype, rope_cos, rope_sin, cache_rows,
                                pos_offset, stream);
}

// ---------------------------------------------------------------------------
// f32 causal attention with materialised probabilities: the computation of
// the reference's per-head CPU attention (crates/prichs-model/src/
// attention.rs:96-149) for one sequence, keeping the [H, T, T] probability
// matrix that the reference's host-slice GPU method returns
// (gpu_batched_attention_forward, crates/prichs-cuda/src/engine.rs:1181-1405).
// One wave per (query row i, head h):
//   s_j = (sum_c q[i][c] k[j][c]) * scale for j <= i (each a sequential sum
//   over c, lanes over j), written into the probability row;
//   m = max_j s_j (exact in any order); e_j = expf(s_j - m);
//   sum of e_j by a fixed wave-tree order; p_j = e_j * (1 / max(sum, 1e-9));
//   zeros past the diagonal; ctx[i][h][c] = sum_j p_j v[j][c] with j
//   ascending (lanes over c).
// ---------------------------------------------------------------------------
namespace prichs {
namespace {
__global__ __launch_bounds__(64) void attn_probs_f32_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    float *__restrict__ probs, float *__restrict__ ctx, int T, int H, int group, int hd,
    float scale) {
#pragma clang fp contract(off)
  extern __shared__ float srow[];  // the row's scores, then probabilities [T]
  const int i = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
  const int kvh = h / group;
  const long long ldq = (long long)H * hd, ldk = (long long)(H / group) * hd;
  const float *qr = q + (long long)i * ldq + (long long)h * hd;
  float mx = -INFINITY;
  for (int j = lane; j <= i; j += 64) {
    const float *kr = k + (long long)j * ldk + (long long)kvh * hd;
    float dot = 0.0f;
    for (int c = 0; c < hd; ++c) {
      const float p = qr[c] * kr[c];
      dot = dot + p;
    }
    const float s = dot * scale;
    srow[j] = s;
    mx = fmaxf(mx, s);
  }
  for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m));
  float sum = 0.0f;
  for (int j = lane; j <= i; j += 64) {
    const float e = expf(srow[j] - mx);
    srow[j] = e;
    sum = sum + e;
  }
  for (int m = 1; m < 64; m <<= 1) sum = sum + __shfl_xor(sum, m);
  const float inv = 1.0f / fmaxf(sum, 1e-9f);
  float *row = probs + ((long long)h * T + i) * T;
  for (int j = lane; j < T; j += 64) {
    const float p = j <= i ? srow[j] * inv : 0.0f;
    if (j <= i) srow[j] = p;
    row[j] = p;
  }
  __syncthreads();  // every lane's probabilities are in LDS
  for (int c = lane; c < hd; c += 64) {
    float acc = 0.0f;
    for (int j = 0; j <= i; ++j) {
      const float p = srow[j] * v[(long long)j * ldk + (long long)kvh * hd + c];
      acc = acc + p;
    }
    ctx[(long long)i * ldq + (long long)h * hd + c] = acc;
  }
}
}  // namespace
}  // namespace prichs

extern "C" int prichs_attention_probs_f32(const float *q, const float *k, const float *v,
                                          float *probs, float *ctx, size_t seq_len,
                                          size_t n_heads, size_t n_kv_heads, size_t head_dim,
                                          void *stream) {
  PRICHS_REQUIRE(n_heads >= 1 && n_kv_heads >= 1 && n_heads % n_kv_heads == 0,
                 "attention_probs: n_heads=%zu must be a positive multiple of n_kv_heads=%zu",
                 n_heads, n_kv_heads);
  PRICHS_REQUIRE(head_dim >= 1 && head_dim <= 65536 && n_heads <= 65535,
                 "attention_probs: shape too large");
  if (seq_len > 16384)
    return fail(PRICHS_ERR_UNSUPPORTED, "attention_probs: seq_len=%zu above 16384 (one row of "
                "scores is kept in LDS)", seq_len);
  if (seq_len == 0) return PRICHS_OK;
  PRICHS_REQUIRE(q && k && v && probs && ctx, "attention_probs: null pointer argument");
  const float scale = 1.0f / sqrtf((float)head_dim);
  hipLaunchKernelGGL(attn_probs_f32_kernel, dim3((unsigned)seq_len, (unsigned)n_heads), dim3(64),
                     seq_len * sizeof(float), as_stream(stream), q, k, v, probs, ctx,
                     (int)seq_len, (int)n_heads,
                     (int)(n_heads / n_kv_heads), (int)head_dim, scale);
  PRICHS_LAUNCH_CHECK("attention_probs launch");
  return PRICHS_OK;
}
