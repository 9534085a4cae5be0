// gemm.hip -- grouped expert GEMMs on CDNA4 MFMA.
//
// Both GEMMs of the MoE FFN run over one "row space": routed rows in the
// permutation order of prichs_permute, then the shared expert's rows.  Group
// g owns rows [offsets[g], offsets[g+1]) and its own weight matrix, so the
// routed experts and the always-on shared expert (a dense group of T rows)
// are one persistent launch: every workgroup walks a global list of
// (group, M-tile, N-tile) tiles, which absorbs skewed routing without
// per-expert launches.
//
//   gate/up:  act[r] = silu(x[row_token[r]] @ Wg) * (x[row_token[r]] @ Wu)
//             (crates/prichs-model/src/moe.rs:166-169, 103-105); the A rows
//             are gathered straight from x, and the gate and up columns of
//             one output column sit in the same lane's accumulators (packed
//             weight interleave), so SwiGLU is applied in the epilogue.
//   down:     y[r] = act[r] @ Wd  (moe.rs:170, 106).
//
// bf16 kernel: 256x256x64 tiles, 8 wave64s in a 2x4 grid each owning a
// 128x64 sub-tile of v_mfma_f32_16x16x32_bf16 accumulators (fp32, two waves
// per SIMD), A and B staged through double-buffered LDS with an XOR swizzle
// of 16-byte chunks, persistent workgroups walking an XCD-aware tile order.
// f32 kernel: 128x128x16 tiles on v_mfma_f32_16x16x4_f32 (the fp32-checked
// mode; accumulates in fp32 like the reference CPU path).
#include <algorithm>
#include <cstring>
#include <vector>

#include "common.hpp"

namespace prichs {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
// Native vector types (not HIP's struct-based uint4/uint2), so staged
// fragments stay in registers.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kMaxGroups = PRICHS_MAX_EXPERTS + 1;
constexpr int kPadRowsDown = 256;  // packed down weights: rows padded to this

// SwiGLU of the bf16 epilogue (silu_ref is the reference formula with the
// full-precision expf and division; silu_fast uses v_exp_f32 / v_rcp_f32).
#ifndef PRICHS_BF16_SILU
#define PRICHS_BF16_SILU silu_fast
#endif
#ifndef PRICHS_BF16_WGM
#define PRICHS_BF16_WGM 2
#endif
#ifndef PRICHS_BF16_WGN
#define PRICHS_BF16_WGN 4
#endif

// ------------------------------------------------------------------------
// Tile scheduler shared by both kernels.
// ------------------------------------------------------------------------
struct TileMap {
  int prefix[kMaxGroups + 1];  // first global M-tile of each group
};

__device__ inline void build_tile_map(TileMap &tm, const int32_t *offsets, int G, int BM) {
  if (threadIdx.x == 0) {
    int run = 0;
    for (int g = 0; g < G; ++g) {
      tm.prefix[g] = run;
      const int mg = offsets[g + 1] - offsets[g];
      run += mg > 0 ? (mg + BM - 1) / BM : 0;
    }
    tm.prefix[G] = run;
  }
  __syncthreads();
}

__device__ inline int find_group(const TileMap &tm, int G, int mt) {
  int g = 0;
  while (g + 1 < G && tm.prefix[g + 1] <= mt) ++g;
  return g;
}

// ------------------------------------------------------------------------
// bf16 kernel
// ------------------------------------------------------------------------
namespace bf {
// Tile shape of one workgroup: BM x BN outputs, K consumed BK at a time.
// WGM x WGN wave64s; a wave owns a WM x WN sub-tile of 16x16 MFMA blocks.
constexpr int BM = 256, BN = 256, BK = 64;
constexpr int WGM = PRICHS_BF16_WGM, WGN = PRICHS_BF16_WGN;
constexpr int kThreads = 64 * WGM * WGN;
constexpr int WM = BM / WGM, WN = BN / WGN;
constexpr int MI = WM / 16, NJ = WN / 16;
constexpr int kIl = WN / 2;             // gate/up interleave: packed blocks [kIl gate | kIl up]
constexpr int kRowsPerPass = kThreads / 8;  // 8 threads load one 128-byte row slice
constexpr int LA = BM / kRowsPerPass;   // A chunks per thread per stage
constexpr int LB = BN / kRowsPerPass;   // B chunks per thread per stage
constexpr int kStageElems = (BM + BN) * BK;
constexpr size_t kLdsBytes = 2 * kStageElems * sizeof(bf16_t);
constexpr int kBandM = 4;               // M-tiles per band of the tile order
static_assert(WN % 32 == 0 && kIl % 16 == 0, "a wave's N sub-tile holds whole gate/up blocks");
static_assert(BN % (2 * kIl) == 0, "packed gate/up rows are padded to a multiple of BN");
static_assert(kRowsPerPass % 8 == 0, "the LDS swizzle key (row & 7) must be pass-invariant");
static_assert(kLdsBytes <= 160 * 1024, "LDS budget of a gfx950 CU");

// LDS element offset of (row, 16-byte chunk) in a [rows][BK] tile; the XOR
// swizzle spreads the 16 rows of one MFMA fragment read over all banks.
__device__ inline int lds_off(int row, int chunk) { return row * BK + ((chunk ^ (row & 7)) << 3); }

// Linear tile id -> (M-tile, N-tile): bands of kBandM M-tiles, N-tiles
// outermost inside a band, so 32 consecutive tiles (one XCD's share of a
// persistent round) touch kBandM A panels and 8 B panels.
__device__ inline void tile_coords(int t, int m_tiles, int n_tiles, int &mt, int &nt) {
  const int band_tiles = kBandM * n_tiles;
  const int band = t / band_tiles;
  const int r = t - band * band_tiles;
  const int rows = min(kBandM, m_tiles - band * kBandM);
  mt = band * kBandM + r % rows;
  nt = r / rows;
}

// C[m, n] = sum_k A[row(m), k] * B[n, k] for the rows of each group, with
// B = packed weights [Np, K] of group g.  The MFMA takes the weight fragment
// as its first operand, so each lane's accumulator holds 4 consecutive
// output columns of one row (D[n][m] of v_mfma_f32_16x16x32_bf16).
template <bool GATEUP>
__global__ __launch_bounds__(kThreads) void grouped_gemm_kernel(
    const bf16_t *__restrict__ A, const int32_t *__restrict__ a_rows, int lda,
    const bf16_t *__restrict__ B, long long b_group_stride, int Np, int K,
    bf16_t *__restrict__ C, int ldc, int n_store, const int32_t *__restrict__ offsets,
    int G) {
  extern __shared__ __attribute__((aligned(16))) bf16_t lds[];
  __shared__ TileMap tm;
  build_tile_map(tm, offsets, G, BM);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WGN, wn = wave - (wave / WGN) * WGN;
  const int n_tiles = Np / BN;
  const int m_tiles = tm.prefix[G];
  const int total = m_tiles * n_tiles;
  const int KT = K / BK;

  const int ld_row = tid >> 3;
  const int ld_chunk = tid & 7;
  const int st_off = lds_off(ld_row, ld_chunk);  // + kRowsPerPass * i * BK per pass i

  const int fr = lane & 15;
  const int a_rd0 = lds_off(wm * WM + fr, lane >> 4);
  const int a_rd1 = lds_off(wm * WM + fr, 4 + (lane >> 4));
  const int b_rd0 = lds_off(wn * WN + fr, lane >> 4);
  const int b_rd1 = lds_off(wn * WN + fr, 4 + (lane >> 4));

  // Workgroups are dealt round-robin to the 8 XCDs; renumber them so each
  // XCD runs a contiguous run of the tile order (shared panels in its L2).
  const int nblk = gridDim.x;
  const int lb = (nblk % 8 == 0) ? (int)(blockIdx.x % 8) * (nblk / 8) + (int)(blockIdx.x / 8)
                                 : (int)blockIdx.x;

  for (int t = lb; t < total; t += nblk) {
    int mt, nt;
    tile_coords(t, m_tiles, n_tiles, mt, nt);
    const int g = find_group(tm, G, mt);
    const int row0 = offsets[g];
    const int mg = offsets[g + 1] - row0;
    const int m0 = (mt - tm.prefix[g]) * BM;
    const int n0 = nt * BN;

    uint32_t a_off[LA];
#pragma unroll
    for (int i = 0; i < LA; ++i) {
      int lr = m0 + ld_row + kRowsPerPass * i;
      lr = lr < mg ? lr : mg - 1;
      const int vr = row0 + lr;
      const int src = a_rows ? a_rows[vr] : vr;
      a_off[i] = (uint32_t)src * (uint32_t)lda + (uint32_t)(ld_chunk * 8);
    }
    const bf16_t *b_base =
        B + (long long)g * b_group_stride + (long long)(n0 + ld_row) * K + ld_chunk * 8;
    const int b_pass = kRowsPerPass * K;

    f32x4 acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    u32x4 ra[LA], rb[LB];
#pragma unroll
    for (int i = 0; i < LA; ++i) ra[i] = *reinterpret_cast<const u32x4 *>(A + a_off[i]);
#pragma unroll
    for (int i = 0; i < LB; ++i) rb[i] = *reinterpret_cast<const u32x4 *>(b_base + i * b_pass);
#pragma unroll
    for (int i = 0; i < LA; ++i)
      *reinterpret_cast<u32x4 *>(lds + st_off + kRowsPerPass * i * BK) = ra[i];
#pragma unroll
    for (int i = 0; i < LB; ++i)
      *reinterpret_cast<u32x4 *>(lds + BM * BK + st_off + kRowsPerPass * i * BK) = rb[i];
    __syncthreads();

    for (int kt = 0; kt < KT; ++kt) {
      const bool more = kt + 1 < KT;
      if (more) {
        const int k0 = (kt + 1) * BK;
#pragma unroll
        for (int i = 0; i < LA; ++i) ra[i] = *reinterpret_cast<const u32x4 *>(A + a_off[i] + k0);
#pragma unroll
        for (int i = 0; i < LB; ++i)
          rb[i] = *reinterpret_cast<const u32x4 *>(b_base + i * b_pass + k0);
      }
      const bf16_t *as = lds + (kt & 1) * kStageElems;
      const bf16_t *bs = as + BM * BK;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        bf16x8 af[MI], wf[NJ];
#pragma unroll
        for (int i = 0; i < MI; ++i)
          af[i] = *reinterpret_cast<const bf16x8 *>(as + (ks ? a_rd1 : a_rd0) + i * 16 * BK);
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          wf[j] = *reinterpret_cast<const bf16x8 *>(bs + (ks ? b_rd1 : b_rd0) + j * 16 * BK);
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int j = 0; j < NJ; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[j], af[i], acc[i][j], 0, 0, 0);
      }
      if (more) {
        bf16_t *as_n = lds + ((kt + 1) & 1) * kStageElems;
#pragma unroll
        for (int i = 0; i < LA; ++i)
          *reinterpret_cast<u32x4 *>(as_n + st_off + kRowsPerPass * i * BK) = ra[i];
#pragma unroll
        for (int i = 0; i < LB; ++i)
          *reinterpret_cast<u32x4 *>(as_n + BM * BK + st_off + kRowsPerPass * i * BK) = rb[i];
      }
      __syncthreads();
    }

    // Epilogue: acc[i][j][r] = C[row m0 + wm*WM + 16i + (lane & 15)]
    //                           [packed col n0 + wn*WN + 16j + 4*(lane >> 4) + r].
    const int lr = m0 + wm * WM + fr;
    const int cq = 4 * (lane >> 4);
    if (GATEUP) {
      // Packed rows [n0 + wn*WN, +WN) are one [kIl gate | kIl up] block:
      // gate column c pairs with up column c in j + NJ/2.
      const int cbase = (n0 + wn * WN) / 2 + cq;
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int m = lr + 16 * i;
        if (m < mg) {
          bf16_t *crow = C + (long long)(row0 + m) * ldc;
#pragma unroll
          for (int j = 0; j < NJ / 2; ++j) {
            const int col = cbase + 16 * j;
            if (col < n_store) {
              uint32_t h[4];
#pragma unroll
              for (int r = 0; r < 4; ++r)
                h[r] = f32_to_bf16(PRICHS_BF16_SILU(acc[i][j][r]) * acc[i][j + NJ / 2][r]);
              *reinterpret_cast<u32x2 *>(crow + col) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
            }
          }
        }
      }
    } else {
      const int cbase = n0 + wn * WN + cq;
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int m = lr + 16 * i;
        if (m < mg) {
          bf16_t *crow = C + (long long)(row0 + m) * ldc;
#pragma unroll
          for (int j = 0; j < NJ; ++j) {
            const int col = cbase + 16 * j;
            if (col < n_store) {
              uint32_t h[4];
#pragma unroll
              for (int r = 0; r < 4; ++r) h[r] = f32_to_bf16(acc[i][j][r]);
              *reinterpret_cast<u32x2 *>(crow + col) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
            }
          }
        }
      }
    }
  }
}
}  // namespace bf

// ------------------------------------------------------------------------
// bf16 kernel, direct-to-LDS pipeline
// ------------------------------------------------------------------------
// Same tile, wave grid, operand order and epilogue as bf::grouped_gemm_kernel;
// the staging differs: global_load_lds_dwordx4 writes each lane's 16 bytes
// straight into LDS (no staging registers, no ds_write), K advances 32 at a
// time through a ring of 4 LDS stages, and loads run 3 stages ahead.  One
// workgroup barrier per stage; waits are explicit vmcnt counts.
namespace bf3 {
constexpr int BM = 256, BN = 256, BK = 32, kStages = 4;
constexpr int WGM = 2, WGN = 4;
constexpr int kThreads = 64 * WGM * WGN;
constexpr int kWaves = WGM * WGN;
constexpr int WM = BM / WGM, WN = BN / WGN;
constexpr int MI = WM / 16, NJ = WN / 16;
constexpr int kIl = WN / 2;
constexpr int kRowsPerInst = 16;  // one wave instruction fills 1 KiB = 16 rows of 64 bytes
constexpr int kInstA = BM / kRowsPerInst / kWaves;
constexpr int kInstB = BN / kRowsPerInst / kWaves;
constexpr int kInstPerStage = kInstA + kInstB;
constexpr int kStageElems = (BM + BN) * BK;
constexpr size_t kLdsBytes = (size_t)kStages * kStageElems * sizeof(bf16_t);
static_assert(kIl == bf::kIl, "both bf16 kernels consume the same packed gate/up layout");
static_assert(BN == bf::BN && BM == bf::BM, "tile shape shared with the register-staged kernel");
static_assert(kInstA * kRowsPerInst * kWaves == BM && kInstB * kRowsPerInst * kWaves == BN,
              "the DMA instructions of one stage cover the A and B tiles exactly");
static_assert(kInstPerStage * 2 <= 63, "vmcnt immediates");
static_assert(kLdsBytes <= 160 * 1024, "LDS budget of a gfx950 CU");

// 64-byte rows of 4 16-byte chunks.  The key makes the 16 rows of one
// fragment read hit distinct banks whether the LDS serves 8 or 16 lanes of a
// ds_read_b128 per cycle.
__device__ inline int swz(int row) { return ((row >> 1) ^ (row >> 2)) & 3; }
__device__ inline int lds_off(int row, int chunk) { return row * BK + ((chunk ^ swz(row)) << 3); }

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] = 7 | lgkmcnt[11:8] = 15 | vmcnt[5:4] at [15:14]).
#define PRICHS_WAIT_VMCNT(n) \
  __builtin_amdgcn_s_waitcnt((((n) & 15) | (((n) >> 4) << 14)) | (7 << 4) | (15 << 8))

__device__ inline void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <bool GATEUP>
__global__ __launch_bounds__(kThreads) void grouped_gemm_kernel(
    const bf16_t *__restrict__ A, const int32_t *__restrict__ a_rows, int lda,
    const bf16_t *__restrict__ B, long long b_group_stride, int Np, int K,
    bf16_t *__restrict__ C, int ldc, int n_store, const int32_t *__restrict__ offsets,
    int G) {
  extern __shared__ __attribute__((aligned(16))) bf16_t lds[];
  __shared__ TileMap tm;
  build_tile_map(tm, offsets, G, BM);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WGN, wn = wave - (wave / WGN) * WGN;
  const int n_tiles = Np / BN;
  const int m_tiles = tm.prefix[G];
  const int total = m_tiles * n_tiles;
  const int KT = K / BK;

  // DMA lane mapping: instruction i of wave w fills rows r0 = 16 (w kInst + i)
  // .. r0 + 15; lane l lands at r0 + l/4, physical chunk l%4, so it loads the
  // logical chunk (l%4) ^ swz(row).
  const int dma_row = lane >> 2;
  const int dma_chunk = (lane & 3) ^ swz(dma_row);  // swz depends on row % 8 only

  const int fr = lane & 15;
  const int a_rd = lds_off(wm * WM + fr, lane >> 4);
  const int b_rd = lds_off(wn * WN + fr, lane >> 4);

  const int nblk = gridDim.x;
  const int lb = (nblk % 8 == 0) ? (int)(blockIdx.x % 8) * (nblk / 8) + (int)(blockIdx.x / 8)
                                 : (int)blockIdx.x;

  for (int t = lb; t < total; t += nblk) {
    int mt, nt;
    bf::tile_coords(t, m_tiles, n_tiles, mt, nt);
    const int g = find_group(tm, G, mt);
    const int row0 = offsets[g];
    const int mg = offsets[g + 1] - row0;
    const int m0 = (mt - tm.prefix[g]) * BM;
    const int n0 = nt * BN;

    uint32_t a_goff[kInstA], b_goff[kInstB];
#pragma unroll
    for (int i = 0; i < kInstA; ++i) {
      int lr = m0 + (wave * kInstA + i) * kRowsPerInst + dma_row;
      lr = lr < mg ? lr : mg - 1;
      const int vr = row0 + lr;
      const int src = a_rows ? a_rows[vr] : vr;
      a_goff[i] = (uint32_t)src * (uint32_t)lda + (uint32_t)(dma_chunk * 8);
    }
#pragma unroll
    for (int i = 0; i < kInstB; ++i) {
      const int nr = n0 + (wave * kInstB + i) * kRowsPerInst + dma_row;
      b_goff[i] = (uint32_t)nr * (uint32_t)K + (uint32_t)(dma_chunk * 8);
    }
    const bf16_t *Bg = B + (long long)g * b_group_stride;

    f32x4 acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // The previous tile's epilogue stores drain and every wave is past its
    // last LDS read before the ring is refilled.
    PRICHS_WAIT_VMCNT(0);
    lds_barrier();

#define PRICHS_ISSUE_STAGE(kt_)                                                       \
  do {                                                                               \
    const int k0_ = (kt_) * BK;                                                      \
    bf16_t *st_ = lds + ((kt_) & (kStages - 1)) * kStageElems;                       \
    _Pragma("unroll") for (int i_ = 0; i_ < kInstA; ++i_)                            \
        __builtin_amdgcn_global_load_lds(A + a_goff[i_] + k0_,                       \
                                         st_ + (wave * kInstA + i_) * kRowsPerInst * BK, \
                                         16, 0, 0);                                  \
    _Pragma("unroll") for (int i_ = 0; i_ < kInstB; ++i_)                            \
        __builtin_amdgcn_global_load_lds(Bg + b_goff[i_] + k0_,                      \
                                         st_ + BM * BK + (wave * kInstB + i_) * kRowsPerInst * BK, \
                                         16, 0, 0);                                  \
  } while (0)

    PRICHS_ISSUE_STAGE(0);
    if (KT > 1) PRICHS_ISSUE_STAGE(1);
    if (KT > 2) PRICHS_ISSUE_STAGE(2);

    for (int kt = 0; kt < KT; ++kt) {
      // Stages issued so far: min(kt + 3, KT); those after kt may stay in flight.
      const int ahead = min(2, KT - 1 - kt);
      if (ahead == 2)
        PRICHS_WAIT_VMCNT(2 * kInstPerStage);
      else if (ahead == 1)
        PRICHS_WAIT_VMCNT(kInstPerStage);
      else
        PRICHS_WAIT_VMCNT(0);
      lds_barrier();
      // The slot refilled here was last read in iteration kt - 1, before the barrier.
      if (kt + 3 < KT) PRICHS_ISSUE_STAGE(kt + 3);

      const bf16_t *as = lds + (kt & (kStages - 1)) * kStageElems;
      const bf16_t *bs = as + BM * BK;
      bf16x8 af[MI], wf[NJ];
#pragma unroll
      for (int i = 0; i < MI; ++i) af[i] = *reinterpret_cast<const bf16x8 *>(as + a_rd + i * 16 * BK);
#pragma unroll
      for (int j = 0; j < NJ; ++j) wf[j] = *reinterpret_cast<const bf16x8 *>(bs + b_rd + j * 16 * BK);
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[j], af[i], acc[i][j], 0, 0, 0);
    }
#undef PRICHS_ISSUE_STAGE

    const int lr = m0 + wm * WM + fr;
    const int cq = 4 * (lane >> 4);
    if (GATEUP) {
      const int cbase = (n0 + wn * WN) / 2 + cq;
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int m = lr + 16 * i;
        if (m < mg) {
          bf16_t *crow = C + (long long)(row0 + m) * ldc;
#pragma unroll
          for (int j = 0; j < NJ / 2; ++j) {
            const int col = cbase + 16 * j;
            if (col < n_store) {
              uint32_t h[4];
#pragma unroll
              for (int r = 0; r < 4; ++r)
                h[r] = f32_to_bf16(PRICHS_BF16_SILU(acc[i][j][r]) * acc[i][j + NJ / 2][r]);
              *reinterpret_cast<u32x2 *>(crow + col) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
            }
          }
        }
      }
    } else {
      const int cbase = n0 + wn * WN + cq;
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int m = lr + 16 * i;
        if (m < mg) {
          bf16_t *crow = C + (long long)(row0 + m) * ldc;
#pragma unroll
          for (int j = 0; j < NJ; ++j) {
            const int col = cbase + 16 * j;
            if (col < n_store) {
              uint32_t h[4];
#pragma unroll
              for (int r = 0; r < 4; ++r) h[r] = f32_to_bf16(acc[i][j][r]);
              *reinterpret_cast<u32x2 *>(crow + col) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
            }
          }
        }
      }
    }
  }
}
}  // namespace bf3

// ------------------------------------------------------------------------
// bf16 kernel, direct-to-LDS pipeline with fragment reads hidden under MFMAs
// ------------------------------------------------------------------------
// Same LDS ring, DMA mapping, tile order and epilogue as bf3.  Each stage's
// MFMAs are split in two halves around the workgroup barrier: after the
// first half frees the A fragments of rows 0..3, the wave waits for the next
// stage, passes the barrier, issues that stage's fragment reads (into the
// freed registers) and the DMA of stage kt + 4, and only then runs the
// second half, so the LDS read latency and bandwidth of one stage overlap the
// MFMAs of the previous one.
namespace bf4 {
using namespace bf3;  // tile shape, swizzle, DMA layout
static_assert(MI % 2 == 0, "two halves of A fragments");

template <bool GATEUP>
__global__ __launch_bounds__(kThreads) void grouped_gemm_kernel(
    const bf16_t *__restrict__ A, const int32_t *__restrict__ a_rows, int lda,
    const bf16_t *__restrict__ B, long long b_group_stride, int Np, int K,
    bf16_t *__restrict__ C, int ldc, int n_store, const int32_t *__restrict__ offsets,
    int G) {
  extern __shared__ __attribute__((aligned(16))) bf16_t lds[];
  __shared__ TileMap tm;
  build_tile_map(tm, offsets, G, BM);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WGN, wn = wave - (wave / WGN) * WGN;
  const int n_tiles = Np / BN;
  const int m_tiles = tm.prefix[G];
  const int total = m_tiles * n_tiles;
  const int KT = K / BK;

  const int dma_row = lane >> 2;
  const int dma_chunk = (lane & 3) ^ swz(dma_row);
  const int fr = lane & 15;
  const int a_rd = lds_off(wm * WM + fr, lane >> 4);
  const int b_rd = lds_off(wn * WN + fr, lane >> 4);

  const int nblk = gridDim.x;
  const int lb = (nblk % 8 == 0) ? (int)(blockIdx.x % 8) * (nblk / 8) + (int)(blockIdx.x / 8)
                                 : (int)blockIdx.x;

  for (int t = lb; t < total; t += nblk) {
    int mt, nt;
    bf::tile_coords(t, m_tiles, n_tiles, mt, nt);
    const int g = find_group(tm, G, mt);
    const int row0 = offsets[g];
    const int mg = offsets[g + 1] - row0;
    const int m0 = (mt - tm.prefix[g]) * BM;
    const int n0 = nt * BN;

    uint32_t a_goff[kInstA], b_goff[kInstB];
#pragma unroll
    for (int i = 0; i < kInstA; ++i) {
      int lr = m0 + (wave * kInstA + i) * kRowsPerInst + dma_row;
      lr = lr < mg ? lr : mg - 1;
      const int vr = row0 + lr;
      const int src = a_rows ? a_rows[vr] : vr;
      a_goff[i] = (uint32_t)src * (uint32_t)lda + (uint32_t)(dma_chunk * 8);
    }
#pragma unroll
    for (int i = 0; i < kInstB; ++i) {
      const int nr = n0 + (wave * kInstB + i) * kRowsPerInst + dma_row;
      b_goff[i] = (uint32_t)nr * (uint32_t)K + (uint32_t)(dma_chunk * 8);
    }
    const bf16_t *Bg = B + (long long)g * b_group_stride;

    f32x4 acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    PRICHS_WAIT_VMCNT(0);
    lds_barrier();

#define PRICHS_ISSUE_STAGE(kt_)                                                       \
  do {                                                                               \
    const int k0_ = (kt_) * BK;                                                      \
    bf16_t *st_ = lds + ((kt_) & (kStages - 1)) * kStageElems;                       \
    _Pragma("unroll") for (int i_ = 0; i_ < kInstA; ++i_)                            \
        __builtin_amdgcn_global_load_lds(A + a_goff[i_] + k0_,                       \
                                         st_ + (wave * kInstA + i_) * kRowsPerInst * BK, \
                                         16, 0, 0);                                  \
    _Pragma("unroll") for (int i_ = 0; i_ < kInstB; ++i_)                            \
        __builtin_amdgcn_global_load_lds(Bg + b_goff[i_] + k0_,                      \
                                         st_ + BM * BK + (wave * kInstB + i_) * kRowsPerInst * BK, \
                                         16, 0, 0);                                  \
  } while (0)

    // Prologue: stages 0..3 in flight; stage 0 lands and is read.
    PRICHS_ISSUE_STAGE(0);
    if (KT > 1) PRICHS_ISSUE_STAGE(1);
    if (KT > 2) PRICHS_ISSUE_STAGE(2);
    if (KT > 3) PRICHS_ISSUE_STAGE(3);
    {
      const int ahead = min(3, KT - 1);  // stages issued after stage 0
      if (ahead == 3)
        PRICHS_WAIT_VMCNT(3 * kInstPerStage);
      else if (ahead == 2)
        PRICHS_WAIT_VMCNT(2 * kInstPerStage);
      else if (ahead == 1)
        PRICHS_WAIT_VMCNT(kInstPerStage);
      else
        PRICHS_WAIT_VMCNT(0);
    }
    lds_barrier();

    bf16x8 af[MI], wf[NJ], wn_next[NJ];
    {
      const bf16_t *as = lds;
      const bf16_t *bs = as + BM * BK;
#pragma unroll
      for (int i = 0; i < MI; ++i) af[i] = *reinterpret_cast<const bf16x8 *>(as + a_rd + i * 16 * BK);
#pragma unroll
      for (int j = 0; j < NJ; ++j) wf[j] = *reinterpret_cast<const bf16x8 *>(bs + b_rd + j * 16 * BK);
    }

    for (int kt = 0; kt < KT; ++kt) {
      // First half: A rows 0 .. MI/2-1 of stage kt.
#pragma unroll
      for (int i = 0; i < MI / 2; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[j], af[i], acc[i][j], 0, 0, 0);

      const bool more = kt + 1 < KT;
      if (more) {
        // Stage kt+1 must have landed; stages kt+2 and kt+3 (if any) may stay in flight.
        const int ahead = min(2, KT - 2 - kt);
        if (ahead == 2)
          PRICHS_WAIT_VMCNT(2 * kInstPerStage);
        else if (ahead == 1)
          PRICHS_WAIT_VMCNT(kInstPerStage);
        else
          PRICHS_WAIT_VMCNT(0);
        lds_barrier();
        // Every wave has read stage kt (in the previous iteration), so its
        // slot takes stage kt + 4.
        if (kt + 4 < KT) PRICHS_ISSUE_STAGE(kt + 4);
        const bf16_t *as = lds + ((kt + 1) & (kStages - 1)) * kStageElems;
        const bf16_t *bs = as + BM * BK;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          wn_next[j] = *reinterpret_cast<const bf16x8 *>(bs + b_rd + j * 16 * BK);
#pragma unroll
        for (int i = 0; i < MI / 2; ++i)
          af[i] = *reinterpret_cast<const bf16x8 *>(as + a_rd + i * 16 * BK);
      }
      // Second half: A rows MI/2 .. MI-1 of stage kt.
#pragma unroll
      for (int i = MI / 2; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[j], af[i], acc[i][j], 0, 0, 0);
      if (more) {
        const bf16_t *as = lds + ((kt + 1) & (kStages - 1)) * kStageElems;
#pragma unroll
        for (int i = MI / 2; i < MI; ++i)
          af[i] = *reinterpret_cast<const bf16x8 *>(as + a_rd + i * 16 * BK);
#pragma unroll
        for (int j = 0; j < NJ; ++j) wf[j] = wn_next[j];
      }
    }
#undef PRICHS_ISSUE_STAGE

    const int lr = m0 + wm * WM + fr;
    const int cq = 4 * (lane >> 4);
    if (GATEUP) {
      const int cbase = (n0 + wn * WN) / 2 + cq;
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int m = lr + 16 * i;
        if (m < mg) {
          bf16_t *crow = C + (long long)(row0 + m) * ldc;
#pragma unroll
          for (int j = 0; j < NJ / 2; ++j) {
            const int col = cbase + 16 * j;
            if (col < n_store) {
              uint32_t h[4];
#pragma unroll
              for (int r = 0; r < 4; ++r)
                h[r] = f32_to_bf16(PRICHS_BF16_SILU(acc[i][j][r]) * acc[i][j + NJ / 2][r]);
              *reinterpret_cast<u32x2 *>(crow + col) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
            }
          }
        }
      }
    } else {
      const int cbase = n0 + wn * WN + cq;
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int m = lr + 16 * i;
        if (m < mg) {
          bf16_t *crow = C + (long long)(row0 + m) * ldc;
#pragma unroll
          for (int j = 0; j < NJ; ++j) {
            const int col = cbase + 16 * j;
            if (col < n_store) {
              uint32_t h[4];
#pragma unroll
              for (int r = 0; r < 4; ++r) h[r] = f32_to_bf16(acc[i][j][r]);
              *reinterpret_cast<u32x2 *>(crow + col) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
            }
          }
        }
      }
    }
  }
}
}  // namespace bf4

// ------------------------------------------------------------------------
// f32 kernel (fp32-checked mode)
// ------------------------------------------------------------------------
namespace fp {
constexpr int BM = 128, BN = 128, BK = 16;
constexpr int kThreads = 256;
constexpr int WM = 64, WN = 64;
constexpr int MI = WM / 16, NJ = WN / 16;
constexpr int kIl = 32;
constexpr int kLd = BK + 1;  // padded LDS row (floats)
constexpr int kStage = (BM + BN) * kLd;
constexpr size_t kLdsBytes = 2 * kStage * sizeof(float);
static_assert(WN == 2 * kIl, "a wave's N sub-tile must hold one gate/up block");
static_assert(BN == 4 * kIl, "packed gate/up rows are padded to a multiple of 4 * il");

template <bool GATEUP>
__global__ __launch_bounds__(kThreads) void grouped_gemm_kernel(
    const float *__restrict__ A, const int32_t *__restrict__ a_rows, int lda,
    const float *__restrict__ B, long long b_group_stride, int Np, int K,
    float *__restrict__ C, int ldc, int n_store, const int32_t *__restrict__ offsets, int G) {
  extern __shared__ float ldsf[];
  __shared__ TileMap tm;
  build_tile_map(tm, offsets, G, BM);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int n_tiles = Np / BN;
  const int total = tm.prefix[G] * n_tiles;
  const int KT = K / BK;
  const int ld_row = tid >> 2;  // + 64*i
  const int ld_c4 = (tid & 3) * 4;

  for (int tile = blockIdx.x; tile < total; tile += gridDim.x) {
    const int mt = tile / n_tiles;
    const int nt = tile - mt * n_tiles;
    const int g = find_group(tm, G, mt);
    const int row0 = offsets[g];
    const int mg = offsets[g + 1] - row0;
    const int m0 = (mt - tm.prefix[g]) * BM;
    const int n0 = nt * BN;
    const float *Bg = B + (long long)g * b_group_stride;
    const float *a_ptr[2];
    const float *b_ptr[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      int lr = m0 + ld_row + 64 * i;
      lr = lr < mg ? lr : mg - 1;
      const int vr = row0 + lr;
      const int src = a_rows ? a_rows[vr] : vr;
      a_ptr[i] = A + (long long)src * lda + ld_c4;
      b_ptr[i] = Bg + (long long)(n0 + ld_row + 64 * i) * K + ld_c4;
    }
    f32x4 acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    float4 ra[2], rb[2];
    auto gload = [&](int k0) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        ra[i] = *reinterpret_cast<const float4 *>(a_ptr[i] + k0);
        rb[i] = *reinterpret_cast<const float4 *>(b_ptr[i] + k0);
      }
    };
    auto lstore = [&](int buf) {
      float *as = ldsf + buf * kStage;
      float *bs = as + BM * kLd;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        float *pa = as + (ld_row + 64 * i) * kLd + ld_c4;
        float *pb = bs + (ld_row + 64 * i) * kLd + ld_c4;
        pa[0] = ra[i].x; pa[1] = ra[i].y; pa[2] = ra[i].z; pa[3] = ra[i].w;
        pb[0] = rb[i].x; pb[1] = rb[i].y; pb[2] = rb[i].z; pb[3] = rb[i].w;
      }
    };
    auto compute = [&](int buf) {
      const float *as = ldsf + buf * kStage;
      const float *bs = as + BM * kLd;
#pragma unroll
      for (int ks = 0; ks < BK / 4; ++ks) {
        const int kk = ks * 4 + (lane >> 4);
        float af[MI], bfr[NJ];
#pragma unroll
        for (int i = 0; i < MI; ++i) af[i] = as[(wm * WM + i * 16 + (lane & 15)) * kLd + kk];
#pragma unroll
        for (int j = 0; j < NJ; ++j) bfr[j] = bs[(wn * WN + j * 16 + (lane & 15)) * kLd + kk];
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int j = 0; j < NJ; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i], bfr[j], acc[i][j], 0, 0, 0);
      }
    };

    gload(0);
    lstore(0);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
      const bool more = kt + 1 < KT;
      if (more) gload((kt + 1) * BK);
      compute(kt & 1);
      if (more) lstore((kt + 1) & 1);
      __syncthreads();
    }

    const int rbase = m0 + wm * WM + 4 * (lane >> 4);
    if (GATEUP) {
      const int cbase = (n0 / (2 * kIl) + wn) * kIl + (lane & 15);
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int lr = rbase + i * 16 + r;
          if (lr < mg) {
            float *crow = C + (long long)(row0 + lr) * ldc;
#pragma unroll
            for (int j = 0; j < NJ / 2; ++j) {
              const int col = cbase + j * 16;
              if (col < n_store) crow[col] = silu_ref(acc[i][j][r]) * acc[i][j + NJ / 2][r];
            }
          }
        }
    } else {
      const int cbase = n0 + wn * WN + (lane & 15);
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int lr = rbase + i * 16 + r;
          if (lr < mg) {
            float *crow = C + (long long)(row0 + lr) * ldc;
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
              const int col = cbase + j * 16;
              if (col < n_store) crow[col] = acc[i][j][r];
            }
          }
        }
    }
  }
}
}  // namespace fp

size_t il_of(int dtype) { return dtype == PRICHS_DTYPE_BF16 ? (size_t)bf::kIl : (size_t)fp::kIl; }
size_t bn_of(int dtype) { return dtype == PRICHS_DTYPE_BF16 ? (size_t)bf::BN : (size_t)fp::BN; }

int check_gemm_shape(size_t d, size_t f, int dtype, const char *who) {
  if (!dtype_ok(dtype)) return fail(PRICHS_ERR_INVALID_ARGUMENT, "%s: bad dtype %d", who, dtype);
  const size_t q = dtype == PRICHS_DTYPE_BF16 ? (size_t)bf::BK : (size_t)fp::BK;
  if (d == 0 || f == 0 || d % q || f % q)
    return fail(PRICHS_ERR_UNSUPPORTED, "%s: d=%zu and f=%zu must be positive multiples of %zu",
                who, d, f, q);
  if (d > (1u << 20) || f > (1u << 20))
    return fail(PRICHS_ERR_UNSUPPORTED, "%s: d=%zu or f=%zu too large", who, d, f);
  return PRICHS_OK;
}

template <typename T> void put(void *out, size_t i, float v);
template <> void put<float>(void *out, size_t i, float v) { static_cast<float *>(out)[i] = v; }
template <> void put<bf16_t>(void *out, size_t i, float v) {
  static_cast<bf16_t *>(out)[i] = f32_to_bf16(v);
}

// Packed gate/up rows: the [il gate | il up] blocks covering f columns,
// padded with zero rows to a multiple of the kernel's N tile.
size_t gate_up_np(size_t f, int dtype) { return roundup(2 * roundup(f, il_of(dtype)), bn_of(dtype)); }

template <typename T>
void pack_gate_up_impl(const float *gate, const float *up, size_t d, size_t f, int dtype,
                       void *out) {
  const size_t il = il_of(dtype);
  const size_t np = gate_up_np(f, dtype);
  for (size_t p = 0; p < np; ++p) {
    const size_t b = p / (2 * il), q = p % (2 * il);
    const float *src = q < il ? gate : up;
    const size_t col = il * b + (q < il ? q : q - il);
    for (size_t k = 0; k < d; ++k) put<T>(out, p * d + k, col < f ? src[k * f + col] : 0.0f);
  }
}

template <typename T> void pack_down_impl(const float *down, size_t d, size_t f, void *out) {
  const size_t np = roundup(d, kPadRowsDown);
  for (size_t n = 0; n < np; ++n)
    for (size_t k = 0; k < f; ++k) put<T>(out, n * f + k, n < d ? down[k * d + n] : 0.0f);
}

#ifndef PRICHS_GEMM_VERSION
#define PRICHS_GEMM_VERSION 4
#endif
#if PRICHS_GEMM_VERSION == 4
namespace BFK = bf4;
#elif PRICHS_GEMM_VERSION == 3
namespace BFK = bf3;
#else
namespace BFK = bf;
#endif

int launch_grouped(bool gateup, const void *A, const int32_t *a_rows, int lda, const void *B,
                   long long b_stride, int Np, int K, void *Cp, int ldc, int n_store,
                   const int32_t *offsets, int G, size_t max_rows, int dtype, hipStream_t s) {
  const int cus = device_cu_count();
  if (cus <= 0) return fail(PRICHS_ERR_HIP, "grouped gemm: cannot query the device");
  if (dtype == PRICHS_DTYPE_BF16) {
    const size_t ub = (max_rows / BFK::BM + G) * (size_t)(Np / BFK::BN);
    const int grid = (int)std::max<size_t>(1, std::min<size_t>(ub, (size_t)cus));
    auto kern = gateup ? BFK::grouped_gemm_kernel<true> : BFK::grouped_gemm_kernel<false>;
    static bool attr_set[2] = {false, false};
    if (!attr_set[gateup]) {
      PRICHS_HIP_TRY(hipFuncSetAttribute((const void *)kern,
                                         hipFuncAttributeMaxDynamicSharedMemorySize,
                                         (int)BFK::kLdsBytes),
                     "grouped gemm: set LDS size");
      attr_set[gateup] = true;
    }
    hipLaunchKernelGGL(kern, dim3(grid), dim3(BFK::kThreads), BFK::kLdsBytes, s,
                       static_cast<const bf16_t *>(A), a_rows, lda,
                       static_cast<const bf16_t *>(B), b_stride, Np, K,
                       static_cast<bf16_t *>(Cp), ldc, n_store, offsets, G);
  } else {
    const size_t ub = (max_rows / fp::BM + G) * (size_t)(Np / fp::BN);
    const int grid = (int)std::max<size_t>(1, std::min<size_t>(ub, (size_t)cus * 4));
    auto kern = gateup ? fp::grouped_gemm_kernel<true> : fp::grouped_gemm_kernel<false>;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(fp::kThreads), fp::kLdsBytes, s,
                       static_cast<const float *>(A), a_rows, lda,
                       static_cast<const float *>(B), b_stride, Np, K,
                       static_cast<float *>(Cp), ldc, n_store, offsets, G);
  }
  PRICHS_LAUNCH_CHECK("grouped gemm launch");
  return PRICHS_OK;
}

}  // namespace
}  // namespace prichs

using namespace prichs;

extern "C" size_t prichs_gate_up_interleave(int dtype) { return dtype_ok(dtype) ? il_of(dtype) : 0; }

extern "C" size_t prichs_packed_gate_up_elems(size_t d, size_t f, int dtype) {
  if (!dtype_ok(dtype)) return 0;
  return gate_up_np(f, dtype) * d;
}

extern "C" size_t prichs_packed_down_elems(size_t d, size_t f, int dtype) {
  if (!dtype_ok(dtype)) return 0;
  return roundup(d, kPadRowsDown) * f;
}

extern "C" int prichs_pack_gate_up(const float *gate, const float *up, size_t d, size_t f,
                                   int dtype, void *packed_out) {
  if (int rc = check_gemm_shape(d, f, dtype, "pack_gate_up")) return rc;
  PRICHS_REQUIRE(gate && up && packed_out, "pack_gate_up: null pointer argument");
  if (dtype == PRICHS_DTYPE_BF16)
    pack_gate_up_impl<bf16_t>(gate, up, d, f, dtype, packed_out);
  else
    pack_gate_up_impl<float>(gate, up, d, f, dtype, packed_out);
  return PRICHS_OK;
}

extern "C" int prichs_pack_down(const float *down, size_t d, size_t f, int dtype,
                                void *packed_out) {
  if (int rc = check_gemm_shape(d, f, dtype, "pack_down")) return rc;
  PRICHS_REQUIRE(down && packed_out, "pack_down: null pointer argument");
  if (dtype == PRICHS_DTYPE_BF16)
    pack_down_impl<bf16_t>(down, d, f, packed_out);
  else
    pack_down_impl<float>(down, d, f, packed_out);
  return PRICHS_OK;
}

extern "C" int prichs_grouped_gate_up_swiglu(const void *x, const int32_t *row_token,
                                             const int32_t *offsets, size_t G, size_t max_rows,
                                             const void *w_packed, size_t d, size_t f, int dtype,
                                             void *act, void *stream) {
  if (int rc = check_gemm_shape(d, f, dtype, "gate_up")) return rc;
  PRICHS_REQUIRE(G >= 1 && G <= (size_t)kMaxGroups, "gate_up: G=%zu outside [1, %d]", G,
                 kMaxGroups);
  PRICHS_REQUIRE(x && row_token && offsets && w_packed && act, "gate_up: null pointer argument");
  PRICHS_REQUIRE(max_rows <= (size_t)INT32_MAX, "gate_up: max_rows too large");
  const size_t np = gate_up_np(f, dtype);
  return launch_grouped(true, x, row_token, (int)d, w_packed, (long long)(np * d), (int)np,
                        (int)d, act, (int)f, (int)f, offsets, (int)G, max_rows, dtype,
                        as_stream(stream));
}

extern "C" int prichs_grouped_down(const void *act, const int32_t *offsets, size_t G,
                                   size_t max_rows, const void *w_packed, size_t d, size_t f,
                                   int dtype, void *y, void *stream) {
  if (int rc = check_gemm_shape(d, f, dtype, "down")) return rc;
  PRICHS_REQUIRE(G >= 1 && G <= (size_t)kMaxGroups, "down: G=%zu outside [1, %d]", G,
                 kMaxGroups);
  PRICHS_REQUIRE(act && offsets && w_packed && y, "down: null pointer argument");
  PRICHS_REQUIRE(max_rows <= (size_t)INT32_MAX, "down: max_rows too large");
  const size_t np = roundup(d, kPadRowsDown);
  return launch_grouped(false, act, nullptr, (int)f, w_packed, (long long)(np * f), (int)np,
                        (int)f, y, (int)d, (int)d, offsets, (int)G, max_rows, dtype,
                        as_stream(stream));
}
