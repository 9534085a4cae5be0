// attention.hip -- causal GQA self-attention forward (flash-style) on CDNA4
// MFMA, for the PrichsBlock attention sub-layer.
//
// Semantics: crates/prichs-model/src/attention.rs:94-149 -- per head h with
// kv head h / (Hq / Hkv): scores = (q . k) * scale over j <= i, softmax over
// the causal row, out = sum_j p_j v_j.  The T x T score matrix is never
// materialised: each workgroup streams 64-row K/V blocks through LDS and
// keeps an online softmax (running max m and partial sums l per query row).
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

__device__ __forceinline__ void dma_16b(const bf16_t *src, bf16_t *lds_dst) {
  __builtin_amdgcn_global_load_lds(src, lds_dst, 16, 0, 0);
}
// ds_read_b64_tr_b16 as inline asm: the builtin form makes the compiler wait
// for every DMA in flight (it cannot tell the read from the DMA's target).
// The result is pending until lds_wait_tied() below, which takes the
// registers as operands so no use can be scheduled before the wait.
__device__ __forceinline__ u32x2 ds_read_tr16(const bf16_t *p) {
  const uint32_t a = (uint32_t)(size_t)(const __attribute__((address_space(3))) bf16_t *)p;
  u32x2 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(r) : "v"(a));
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

// q/k/v/o: row r of sequence b is row b*S + r; head h of q/o starts at column
// h*128, kv head j of k/v at column j*128 (leading dimensions ldq/ldk/ldv/ldo).
template <int HPW>
__global__ __launch_bounds__(kThreads, 2) void attn_fwd_kernel(
    const bf16_t *__restrict__ q, int ldq, const bf16_t *__restrict__ k, int ldk,
    const bf16_t *__restrict__ v, int ldv, bf16_t *__restrict__ o, int ldo, int S, int Hq,
    int group, float scale_log2) {
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
  const int wave = tid >> 6;
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
  }

  f32x4 oacc[8][2];  // O^T blocks: d block jd, query block nb
#pragma unroll
  for (int jd = 0; jd < 8; ++jd)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) oacc[jd][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run[2] = {-INFINITY, -INFINITY};  // running max (log2 units) of row q
  float l_part[2] = {0.f, 0.f};              // this lane's share of the row sum

  // kv blocks up to the last query row of the workgroup (causal).
  const int q_last = min(S, (qb + 1) * kRowsWg) - 1;
  const int n_kvb = q_last / kBKV + 1;

  // DMA of one K/V block into stage buffer `st`: wave w moves rows
  // 16 w .. 16 w + 15 of each tile, 4 rows (1 KiB) per instruction; the lane
  // for LDS slot (row, s) fetches logical chunk s ^ key(row).  Rows past the
  // sequence repeat its last row (their scores are masked).
  auto issue_block = [&](int kb, int st) {
    bf16_t *kst = lds + st * kStageElems;
    bf16_t *vst = kst + kTileElems;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * wave + 4 * i + (lane >> 4);
      const int slot = lane & 15;
      const int src = min(kb * kBKV + row, S - 1);
      const int base = (16 * wave + 4 * i) * kHd;  // wave-uniform LDS destination
      dma_16b(kbase + (size_t)src * ldk + 8 * (slot ^ k_key(row)), kst + base);
      dma_16b(vbase + (size_t)src * ldv + 8 * (slot ^ v_key(row)), vst + base);
    }
  };
  issue_block(0, 0);

  for (int kb = 0; kb < n_kvb; ++kb) {
    const int kv0 = kb * kBKV;
    const bf16_t *ks = lds + (kb & 1) * kStageElems;
    const bf16_t *vs = ks + kTileElems;
    // This block's tiles have landed (every wave waits for its own DMA, the
    // barrier for the others'), and every wave is done with the other stage
    // buffer (block kb - 1), which now takes block kb + 1.
    // s_waitcnt vmcnt(0) (gfx9 encoding: vmcnt[3:0] | expcnt 7 << 4 |
    // lgkmcnt 15 << 8 | vmcnt[5:4] << 14).
    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
    __syncthreads();
    if (kb + 1 < n_kvb) issue_block(kb + 1, (kb + 1) & 1);

    // S^T = K Q^T for 4 kv blocks x 2 query blocks.
    f32x4 st[4][2];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) st[c][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      bf16x8 kf[4];
#pragma unroll
      for (int c = 0; c < 4; ++c)
        kf[c] = *reinterpret_cast<const bf16x8 *>(ks + k_off(16 * c + l16, 4 * kk + g));
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) st[c][nb] = mfma_bf16(kf[c], qf[nb][kk], st[c][nb]);
    }

    // Online softmax.  st[c][nb][r] = score of (query q0 + 16nb + l16,
    // kv kv0 + 16c + 4g + r).
    u32x4 pf[2][2];  // P fragments: [nb][32-row kv step]
    // Only blocks reaching past this wave's first query row or the sequence
    // end need the causal / length mask (wave-uniform test).
    const bool masked = kv0 + kBKV - 1 > q0 || kv0 + kBKV > S;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int qrow = q0 + 16 * nb + l16;
      float s[16];
      float mloc = -INFINITY;
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int kv = kv0 + 16 * c + 4 * g + r;
          float x = st[c][nb][r] * scale_log2;
          if (masked) x = (kv <= qrow && kv < S) ? x : -INFINITY;
          s[4 * c + r] = x;
          mloc = fmaxf(mloc, x);
        }
      mloc = fmaxf(mloc, __shfl_xor(mloc, 16, 64));
      mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
      const float m_new = fmaxf(m_run[nb], mloc);
      // Rows with no valid score yet keep m = -inf; exp2(-inf - -inf) would be NaN.
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = fast_exp2(m_run[nb] - m_use);
      m_run[nb] = m_new;
      float psum = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float p = fast_exp2(s[i] - m_use);
        s[i] = p;
        psum += p;
      }
      l_part[nb] = l_part[nb] * alpha + psum;
      // Rescale the output rows only when some row's running max moved
      // (alpha == 1 exactly otherwise, so skipping changes nothing).
      if (__any(alpha != 1.0f)) {
#pragma unroll
        for (int jd = 0; jd < 8; ++jd) oacc[jd][nb] = oacc[jd][nb] * alpha;
      }
#pragma unroll
      for (int ks2 = 0; ks2 < 2; ++ks2) {
        // k slots 0..3: kv block 2 ks2 (rows 4g + r); slots 4..7: block 2 ks2 + 1.
        const float *a0 = s + 4 * (2 * ks2);
        const float *a1 = s + 4 * (2 * ks2 + 1);
        pf[nb][ks2] = u32x4{pack_bf16(a0[0], a0[1]), pack_bf16(a0[2], a0[3]),
                            pack_bf16(a1[0], a1[1]), pack_bf16(a1[2], a1[3])};
      }
    }

    // O^T += V^T P^T: d blocks jd, 32-row kv steps ks2.
#pragma unroll
    for (int ks2 = 0; ks2 < 2; ++ks2) {
      // Lane m of each 16-lane group reads row r0 + m/4 (r0 = 32 ks2 + 4 g, and
      // 16 rows on for the upper half), columns 16 jd + 4 (m % 4) .. + 3;
      // four d blocks per batch of transposing reads.
      const int vr = 32 * ks2 + 4 * g + (l16 >> 2);
      const int ve = 4 * (l16 & 3);  // element within the 16-column block
#pragma unroll
      for (int j0 = 0; j0 < 8; j0 += 4) {
        u32x2 lo[4], hi[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int col = 16 * (j0 + t) + ve;
          lo[t] = ds_read_tr16(vs + v_off(vr, col >> 3) + (col & 7));
          hi[t] = ds_read_tr16(vs + v_off(vr + 16, col >> 3) + (col & 7));
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
    }
  }

  // Normalise by the row sum and store: lane holds O[q][16 jd + 4g + r].
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    float l = l_part[nb];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const float inv = 1.0f / fmaxf(l, 1e-30f);
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

extern "C" int prichs_attention_forward(const void *q, size_t ldq, const void *k, size_t ldk,
                                        const void *v, size_t ldv, void *o, size_t ldo,
                                        size_t batch, size_t seq_len, size_t n_heads,
                                        size_t n_kv_heads, size_t head_dim, int dtype,
                                        void *stream) {
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
                     ldq <= (size_t)INT32_MAX && ldk <= (size_t)INT32_MAX &&
                     ldv <= (size_t)INT32_MAX && ldo <= (size_t)INT32_MAX,
                 "attention: shape too large");
  if (batch == 0 || seq_len == 0) return PRICHS_OK;
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
                     scale_log2);
  PRICHS_LAUNCH_CHECK("attention launch");
  return PRICHS_OK;
}
