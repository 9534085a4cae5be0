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
// bf16 kernel: 256x256 output tiles per workgroup (8 waves of 64x128) on
// v_mfma_f32_16x16x32_bf16 (fp32 accumulation).  K advances 32 at a time
// through a ring of 4 LDS stages that global_load_lds_dwordx4 fills directly
// (no staging registers), 3 stages ahead of the MFMAs; the two halves of the
// workgroup ping-pong, one wave per SIMD multiplying while the other reads
// its fragments and issues loads.  Workgroups are persistent and walk an
// XCD-aware tile order.  The epilogues stage the finished tile in LDS and
// write whole rows with 16-byte lanes (down / dense: the tile; gate/up: the
// activations, or in the training forward the pre-activations, whose
// activations then exchange halves between lane pairs and write 16 bytes per
// lane).
// f32 kernel: 128x128x16 tiles on v_mfma_f32_16x16x4_f32 (the fp32-checked
// mode; accumulates in fp32 like the reference CPU path).
#include <algorithm>
#include <cstdlib>
#include <type_traits>
#include <cstring>
#include <vector>

#include "common.hpp"
#include "router_quad.hpp"

namespace prichs {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
// Native vector types (not HIP's struct-based uint4/uint2), so values stay
// in registers.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
template <bool B> using bool_c = std::integral_constant<bool, B>;

constexpr int kMaxGroups = PRICHS_MAX_EXPERTS + 1;
constexpr int kPadRowsDown = 256;    // packed down weights: rows padded to this
constexpr int kBf16KMultiple = 64;   // bf16 kernels need d and f to be multiples of this

// SwiGLU of the bf16 epilogue (silu_ref is the reference formula with the
// full-precision expf and division; silu_fast uses v_exp_f32 / v_rcp_f32).
#ifndef PRICHS_BF16_SILU
#define PRICHS_BF16_SILU silu_fast
#endif
// Wave grids of the bf16 kernel (WGM x WGN wave64s per tile): 256 x 256
// tiles as 4 x 2 waves of 64 x 128 (against 2 x 4 waves of 128 x 64, the same
// LDS bytes per MFMA: config 2 gate/up 155.6 -> 155.0 us, down 98.6 -> 98.1,
// and 2.4 / 2.8 us less after an L2/MALL flush); the 128 x 384 tiles keep
// 2 x 4 waves of 64 x 96.
#ifndef PRICHS_BF16_WGM
#define PRICHS_BF16_WGM 4
#endif
#ifndef PRICHS_BF16_WGN
#define PRICHS_BF16_WGN 2
#endif
// Down / dense epilogue through an LDS copy of the tile with 16-byte row
// stores (1) or direct 8-byte stores from the accumulators (0).
#ifndef PRICHS_GEMM_STAGE_C
#define PRICHS_GEMM_STAGE_C 1
#endif
// M-tiles per band of the tile order.
#ifndef PRICHS_BAND_M
#define PRICHS_BAND_M 4
#endif

// ------------------------------------------------------------------------
// Tile scheduler shared by the kernels.
// ------------------------------------------------------------------------
struct TileMap {
  int prefix[kMaxGroups + 1];  // first global M-tile of each group
  int offs[kMaxGroups + 1];    // offsets[] of the launch (row range of each group)
};

// offsets == nullptr is the dense case: one group of dense_m rows (G == 1).
__device__ inline void build_tile_map(TileMap &tm, const int32_t *offsets, int G, int BM,
                                      int dense_m) {
  if (threadIdx.x == 0 && offsets == nullptr) {
    tm.prefix[0] = 0;
    tm.offs[0] = 0;
    tm.prefix[1] = (dense_m + BM - 1) / BM;
    tm.offs[1] = dense_m;
  } else if (threadIdx.x == 0) {
    int run = 0;
    for (int g = 0; g < G; ++g) {
      tm.prefix[g] = run;
      tm.offs[g] = offsets[g];
      const int mg = offsets[g + 1] - offsets[g];
      run += mg > 0 ? (mg + BM - 1) / BM : 0;
    }
    tm.prefix[G] = run;
    tm.offs[G] = offsets[G];
  }
  __syncthreads();
}

// The same table held in registers by every wave of a launch (the bf16
// kernels' LDS is all ring): entry e <= G -- the first global M-tile (prefix)
// and first row (offs) of group e -- sits in lane e % 64 of word e / 64.
struct WaveTileMap {
  int prefix[2], offs[2];
  int G, m_tiles;
};

__device__ inline void build_wave_tile_map(WaveTileMap &tm, const int32_t *offsets, int G,
                                           int BM, int dense_m) {
  static_assert(kMaxGroups + 1 <= 128, "two words per lane hold the group table");
  const int lane = threadIdx.x & 63;
  tm.G = G;
  int carry = 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int e = 64 * h + lane;
    int off, next;
    if (offsets == nullptr) {  // dense: one group of dense_m rows
      off = e == 0 ? 0 : dense_m;
      next = dense_m;
    } else {
      off = offsets[min(e, G)];
      next = offsets[min(e + 1, G)];
    }
    const int tiles = (e < G && next > off) ? (next - off + BM - 1) / BM : 0;
    int inc = tiles;  // inclusive scan over the wave
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int t = __shfl_up(inc, d);
      if (lane >= d) inc += t;
    }
    tm.prefix[h] = carry + inc - tiles;
    tm.offs[h] = off;
    carry += __shfl(inc, 63);
  }
  tm.m_tiles = carry;
}

// Entry e (wave-uniform) of one of the two-word tables.
__device__ __forceinline__ int wave_entry(const int (&w)[2], int e) {
  return e < 64 ? __builtin_amdgcn_readlane(w[0], e) : __builtin_amdgcn_readlane(w[1], e - 64);
}

// Group of global M-tile mt: the number of groups e in [1, G) whose first
// M-tile is <= mt (prefix is nondecreasing; empty groups own no tiles).
__device__ __forceinline__ int wave_find_group(const WaveTileMap &tm, int mt) {
  const int lane = threadIdx.x & 63;
  const unsigned long long b0 = __ballot(lane >= 1 && lane < tm.G && tm.prefix[0] <= mt);
  const unsigned long long b1 = __ballot(64 + lane < tm.G && tm.prefix[1] <= mt);
  return __builtin_amdgcn_readfirstlane(__popcll(b0) + __popcll(b1));
}

// Group of global M-tile mt (empty groups own no tiles and are skipped).
__device__ inline int find_group(const TileMap &tm, int G, int mt) {
  int g = 0;
  while (g + 1 < G && tm.prefix[g + 1] <= mt) ++g;
  return g;
}

// Linear tile id -> (M-tile, N-tile): bands of PRICHS_BAND_M M-tiles with the
// N-tiles outermost inside a band, so a run of consecutive tiles shares a few
// A panels and B panels.
__device__ inline void tile_coords(int t, int m_tiles, int n_tiles, int &mt, int &nt) {
  const int band_tiles = PRICHS_BAND_M * n_tiles;
  const int band = t / band_tiles;
  const int r = t - band * band_tiles;
  const int rows = min(PRICHS_BAND_M, m_tiles - band * PRICHS_BAND_M);
  mt = band * PRICHS_BAND_M + r % rows;
  nt = r / rows;
}

// Workgroups are dealt round-robin to the 8 XCDs; renumbering them so each XCD
// runs a contiguous run of the tile order keeps shared panels in its L2.
__device__ inline int xcd_block_id() {
  const int nblk = gridDim.x;
  return (nblk % 8 == 0) ? (int)(blockIdx.x % 8) * (nblk / 8) + (int)(blockIdx.x / 8)
                         : (int)blockIdx.x;
}

// ------------------------------------------------------------------------
// bf16 kernel
// ------------------------------------------------------------------------
// LDS stage layout: [rows][32] bf16, 64-byte rows of 4 16-byte chunks.  The
// XOR key makes the 16 rows of one fragment read hit distinct banks whether
// the LDS serves 8 or 16 lanes of a ds_read_b128 per cycle.
constexpr int kBK = 32;
__device__ inline int swz(int row) { return ((row >> 1) ^ (row >> 2)) & 3; }
__device__ inline int lds_off(int row, int chunk) { return row * kBK + ((chunk ^ swz(row)) << 3); }

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] = 7 | lgkmcnt[11:8] = 15 | vmcnt[5:4] at [15:14]).
#define PRICHS_WAIT_VMCNT(n) \
  __builtin_amdgcn_s_waitcnt((((n) & 15) | (((n) >> 4) << 14)) | (7 << 4) | (15 << 8))

// Non-template wrappers of the target builtins: a builtin call whose
// arguments depend on a kernel template parameter fails (silently) in the
// host compilation pass, which then emits no host stub for the kernel.
__device__ __forceinline__ void wait_vmcnt(int n) {
  switch (n) {
#define PRICHS_VMCNT_CASE(v) \
  case v:                    \
    PRICHS_WAIT_VMCNT(v);    \
    break;
    PRICHS_VMCNT_CASE(0) PRICHS_VMCNT_CASE(1) PRICHS_VMCNT_CASE(2) PRICHS_VMCNT_CASE(3)
    PRICHS_VMCNT_CASE(4) PRICHS_VMCNT_CASE(5) PRICHS_VMCNT_CASE(6) PRICHS_VMCNT_CASE(7)
    PRICHS_VMCNT_CASE(8) PRICHS_VMCNT_CASE(9) PRICHS_VMCNT_CASE(10) PRICHS_VMCNT_CASE(11)
    PRICHS_VMCNT_CASE(12) PRICHS_VMCNT_CASE(15) PRICHS_VMCNT_CASE(16) PRICHS_VMCNT_CASE(18)
    PRICHS_VMCNT_CASE(20) PRICHS_VMCNT_CASE(24)
#undef PRICHS_VMCNT_CASE
    default:
      PRICHS_WAIT_VMCNT(0);  // any other count: wait for everything (always safe)
      break;
  }
}
__device__ __forceinline__ void dma_16b(const bf16_t *src, bf16_t *lds_dst) {
  __builtin_amdgcn_global_load_lds(src, lds_dst, 16, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_bf16(bf16x8 w, bf16x8 a, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(w, a, c, 0, 0, 0);
}

template <int... Is, class F>
__device__ __forceinline__ void static_for(std::integer_sequence<int, Is...>, F &&f) {
  (f(std::integral_constant<int, Is>{}), ...);
}

// Workgroup barrier without a memory fence: LDS-DMA completion is tracked by
// the explicit vmcnt waits, and a fence would force vmcnt(0).
__device__ inline void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

#ifndef PRICHS_BF16_STAGES
#define PRICHS_BF16_STAGES 4
#endif
template <int BM_, int BN_, int WGM_, int WGN_, int S_ = PRICHS_BF16_STAGES> struct Bf16Cfg {
  static constexpr int BM = BM_, BN = BN_, BK = kBK, kStages = S_;
  static constexpr int WGM = WGM_, WGN = WGN_;
  static constexpr int kWaves = WGM * WGN;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int WM = BM / WGM, WN = BN / WGN;
  static constexpr int MI = WM / 16, NJ = WN / 16;
  static constexpr int kIl = 32;             // gate/up interleave: packed blocks [kIl gate | kIl up]
  static constexpr int kRowsPerInst = 16;    // one wave instruction fills 1 KiB = 16 rows of 64 B
  // DMA instructions of one stage: one per 16-row block of A and of B.  When
  // a count is a multiple of the waves, wave w moves blocks w kInst ..
  // (w + 1) kInst - 1; otherwise blocks are dealt round-robin (block i kWaves
  // + w), so some waves issue one more.  kInstA / kInstB are the per-wave
  // maxima; kInstPerStage, which sets the waits, is the per-wave MINIMUM:
  // vector-memory operations complete in issue order, so allowing only that
  // many of the newest instructions per stage in flight waits for at least
  // as much as a wave needs.
  static constexpr int kBlkA = BM / kRowsPerInst, kBlkB = BN / kRowsPerInst;
  static constexpr bool kEvenA = kBlkA % kWaves == 0, kEvenB = kBlkB % kWaves == 0;
  static constexpr int kInstA = (kBlkA + kWaves - 1) / kWaves;
  static constexpr int kInstB = (kBlkB + kWaves - 1) / kWaves;
  static constexpr int kInstPerStage = kBlkA / kWaves + kBlkB / kWaves;
  static constexpr int kStageElems = (BM + BN) * BK;
  static constexpr size_t kRingBytes = (size_t)kStages * kStageElems * sizeof(bf16_t);
  // Epilogue staging of a finished tile: [BM][BN + 8] bf16 (16-byte row pad)
  // in the ring's LDS, which no wave reads any more by then.
  static constexpr int kStgStride = BN + 8;
  static constexpr size_t kStgBytes = (size_t)BM * kStgStride * sizeof(bf16_t);
  static constexpr size_t kLdsBytes = kRingBytes > kStgBytes ? kRingBytes : kStgBytes;
  static_assert(MI % 2 == 0 && WN % 16 == 0, "two A halves and whole fragments per wave");
  static_assert(kBlkA * kRowsPerInst == BM && kBlkB * kRowsPerInst == BN,
                "the DMA instructions of one stage cover the A and B tiles exactly");
  static_assert(kInstPerStage >= 1, "every wave issues DMA in every stage");
  static_assert(kStages >= 3 && (kStages - 1) * (kInstA + kInstB) <= 63, "vmcnt immediates");
  static_assert(kLdsBytes <= 160 * 1024, "LDS budget of a gfx950 CU");
};
// gate/up: 256x256 tiles; down: PRICHS_DOWN_BM x 256 tiles (smaller M tiles
// spread the down GEMM's fewer tiles more evenly over the CUs).
#ifndef PRICHS_DOWN_BM
#define PRICHS_DOWN_BM 256
#endif
#ifndef PRICHS_DOWN_BN
#define PRICHS_DOWN_BN 256
#endif
using Bf16 = Bf16Cfg<256, 256, PRICHS_BF16_WGM, PRICHS_BF16_WGN>;
using Bf16Down = Bf16Cfg<PRICHS_DOWN_BM, PRICHS_DOWN_BN, PRICHS_BF16_WGM, PRICHS_BF16_WGN>;
static_assert(Bf16::BN % Bf16Down::BN == 0,
              "packed weights are padded to Bf16::BN rows, a whole number of down N tiles");
// Dense (single-group) launches whose padded N is a multiple of 384 may use
// 128 x 384 tiles instead: three quarters of a 256 x 256 tile's work, and a
// tile count that can fill the CUs where 256 x 256 tiles leave a round part
// empty (8192 x 1536 outputs: 256 such tiles against 192).  Each output
// element is the same MFMA chain over K either way, so the bits are the same.
using Bf16Wide = Bf16Cfg<128, 384, 2, 4>;
// ... and launches whose padded N is a multiple of 288 may use 256 x 288
// tiles (8 waves of 64 x 144; 18 B blocks per stage dealt unevenly): the
// block's q/k/v projection (8192 x 2304) is then exactly 256 tiles, one
// round of the CUs, where 256 x 256 tiles make 1.125 rounds and 128 x 384
// tiles 1.5.
using Bf16Tall = Bf16Cfg<256, 288, 4, 2>;

// C[m, n] = sum_k A[row(m), k] * B[n, k] for the rows of each group, with
// B = packed weights [Np, K] of group g.  The MFMA takes the weight fragment
// as its first operand, so each lane's accumulator holds 4 consecutive
// output columns of one row (D[n][m] of v_mfma_f32_16x16x32_bf16), stored as
// one 8-byte write.
// Both bf16 configurations run the same number of waves, so the launch bound
// is a constant (a bound that depends on a template parameter fails to
// substitute in the host pass).
constexpr int kBf16Threads = 64 * PRICHS_BF16_WGM * PRICHS_BF16_WGN;

// Group g's A rows row0.. read from A + delta (elements) instead: the MoE
// backward's dA takes the shared expert's rows of dY from d_out itself.
// g = -1: none.
struct A2Rows {
  long long delta = 0;
  int g = -1, row0 = 0;
};

// One output tile of the grouped GEMM: M-tile mt (global over the groups of
// tm) and N-tile nt of width Cf::BN, computed by the whole workgroup.
// DSW (down configurations only): the tile is dA of the MoE backward and its
// epilogue is the SwiGLU backward: P is then the packed gate/up
// pre-activations [rows][ldc] (ldc = their packed width Np_gu), updated in
// place to dG, dU for the tile's activation columns (n_store = f valid ones;
// those up to Np_gu / 2 beyond f are cleared), and C is not written.
template <class Cf, bool GATEUP, bool DSW = false>
__device__ __forceinline__ void bf16_tile(
    const bf16_t *__restrict__ A, const int32_t *__restrict__ a_rows, int lda,
    const bf16_t *__restrict__ B, long long b_group_stride, int Np, int K,
    bf16_t *__restrict__ C, int ldc, int n_store, const WaveTileMap &tm, int stage_c,
    bf16_t *__restrict__ P, bf16_t *lds, int mt, int nt, const A2Rows &a2) {
  constexpr int BM = Cf::BM, BN = Cf::BN, BK = Cf::BK, kStages = Cf::kStages;
  constexpr int WGN = Cf::WGN, WM = Cf::WM, WN = Cf::WN, MI = Cf::MI, NJ = Cf::NJ;
  constexpr int kRowsPerInst = Cf::kRowsPerInst, kInstA = Cf::kInstA, kInstB = Cf::kInstB;
  constexpr int kInstPerStage = Cf::kInstPerStage, kStageElems = Cf::kStageElems;
  static_assert(Cf::kThreads == kBf16Threads, "launch bound of the bf16 kernels");
  static_assert(Cf::kWaves == 8, "ping-pong K loop: two groups of 4 waves, one of each per SIMD");
  static_assert(!(GATEUP && DSW), "the SwiGLU-backward epilogue is a down / dense mode");
  static_assert(!GATEUP || (WN % (2 * Cf::kIl) == 0 && BN % (2 * Cf::kIl) == 0),
                "whole [gate | up] blocks per wave; packed gate/up rows padded to BN");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN, wn = wave - (wave / WGN) * WGN;
  const int KT = K / BK;

  // DMA lane mapping: instruction i of wave w fills rows r0 = 16 (w kInst + i)
  // .. r0 + 15; lane l lands at row r0 + l/4, physical chunk l%4, so it loads
  // the logical chunk (l%4) ^ swz(row) (swz depends on row % 8 only).
  const int dma_row = lane >> 2;
  const int dma_chunk = (lane & 3) ^ swz(dma_row);

  // Fragment reads: lane l reads row l%16 of a 16-row block, chunk l/16.
  const int fr = lane & 15;
  const int a_rd = lds_off(wm * WM + fr, lane >> 4);
  // B stage: whole packed fragments in weight order, lane-major (1 KiB each).
  const int b_rd = wn * WN * BK + lane * 8;

  const int g = wave_find_group(tm, mt);
  const int row0 = wave_entry(tm.offs, g);
  const int mg = wave_entry(tm.offs, g + 1) - row0;
  const int m0 = (mt - wave_entry(tm.prefix, g)) * BM;
  const int n0 = nt * BN;

  // A offsets are 64-bit (gathered rows: src * lda can pass 2^32 elements for
  // a large row space); B offsets stay within one group's packed weights,
  // which the host bounds to 2^32 elements.
  // 16-row block of DMA instruction i of this wave (see Bf16Cfg), and
  // whether the wave issues that instruction at all (uneven deals).
  auto blk_a = [&](int i) { return Cf::kEvenA ? wave * kInstA + i : i * Cf::kWaves + wave; };
  auto blk_b = [&](int i) { return Cf::kEvenB ? wave * kInstB + i : i * Cf::kWaves + wave; };
  auto has_a = [&](int i) { return Cf::kEvenA || blk_a(i) < Cf::kBlkA; };
  auto has_b = [&](int i) { return Cf::kEvenB || blk_b(i) < Cf::kBlkB; };
  long long a_goff[kInstA];
  uint32_t b_goff[kInstB];
#pragma unroll
  for (int i = 0; i < kInstA; ++i) {
    int lr = m0 + min(blk_a(i), Cf::kBlkA - 1) * kRowsPerInst + dma_row;
    lr = lr < mg ? lr : mg - 1;  // rows past the group repeat its last row
    const int vr = row0 + lr;
    const int src = a_rows ? a_rows[vr] : vr;
    a_goff[i] = g == a2.g ? a2.delta + (long long)(vr - a2.row0) * lda + dma_chunk * 8
                          : (long long)src * lda + dma_chunk * 8;
  }
#pragma unroll
  for (int i = 0; i < kInstB; ++i) {
    // Instruction i moves fragment (16-row block nb, K-step kt): 1 KiB at
    // (nb * KT + kt) * 512 elements, lane l's 16 bytes at l * 8.
    const int nb = n0 / kRowsPerInst + min(blk_b(i), Cf::kBlkB - 1);
    b_goff[i] = (uint32_t)nb * (uint32_t)KT * 512u + (uint32_t)(lane * 8);
  }
  const bf16_t *Bg = B + (long long)g * b_group_stride;

  f32x4 acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // The previous tile's stores drain and every wave is past its last LDS
  // read before the ring is refilled.
  wait_vmcnt(0);
  lds_barrier();

  // DMA instruction `which` of stage kt_: A rows first, then B fragments.
  auto issue_one = [&](int kt_, int which) {
    bf16_t *st_ = lds + (kt_ % kStages) * kStageElems;
    if (which < kInstA) {
      if (has_a(which))
        dma_16b(A + a_goff[which] + kt_ * BK, st_ + blk_a(which) * kRowsPerInst * BK);
    } else {
      const int i_ = which - kInstA;
      if (has_b(i_))
        dma_16b(Bg + b_goff[i_] + kt_ * 512, st_ + BM * BK + blk_b(i_) * kRowsPerInst * BK);
    }
  };
  auto issue_stage = [&](int kt_) {
#pragma unroll
    for (int w = 0; w < kInstA + kInstB; ++w) issue_one(kt_, w);
  };

  // Ping-pong K loop over a ring of S = kStages LDS stages, S - 1 of them in
  // flight.  Waves 0-3 (group 0) and 4-7 (group 1) sit one per SIMD each, so
  // every SIMD hosts one wave of each group.  Every wave runs the same
  // sequence per K-step kt -- a memory phase (read its fragments of stage kt
  // from LDS, issue its share of stage kt + S - 1, wait for its share of
  // stage kt + 1 and for its own LDS reads), a barrier, an MFMA phase on
  // those fragments, a barrier -- but group 1 starts one barrier late, so on
  // each SIMD one wave issues MFMAs while the other does its LDS reads and
  // DMA, and they swap at every barrier: between barriers b(2kt) and
  // b(2kt+1) group 0 multiplies stage kt while group 1 reads it; between
  // b(2kt+1) and b(2kt+2) group 1 multiplies it while group 0 reads stage
  // kt + 1.
  //  - Stage s is first read after b(2s-1); both groups waited for their
  //    shares of it in their memory phases of step s - 1, which end at b(2s-2)
  //    and b(2s-1).
  //  - The share of stage kt + S - 1 issued in step kt's memory phase goes to
  //    stage kt - 1's slot; both groups' LDS reads of stage kt - 1 completed
  //    before b(2kt-2) and b(2kt-1), and step kt's memory phases start after
  //    b(2kt-1) and b(2kt).
  // Each output element is the same MFMA chain over K whatever the
  // schedule, so the results are bit-identical.
  const int grp = wave >> 2;
  // Barrier that nothing is scheduled across (MFMAs touch no memory, so the
  // memory clobber alone would let the scheduler move them over it).
  auto pp_barrier = [] {
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
  };
  struct Frags {
    bf16x8 w[NJ], a[MI];
  } F;
  auto read_frags = [&](int st) {
    const bf16_t *as = lds + (st % kStages) * kStageElems;
    const bf16_t *bs = as + BM * BK;
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj)
      F.w[jj] = *reinterpret_cast<const bf16x8 *>(bs + b_rd + jj * 16 * BK);
#pragma unroll
    for (int ii = 0; ii < MI; ++ii)
      F.a[ii] = *reinterpret_cast<const bf16x8 *>(as + a_rd + ii * 16 * BK);
  };
  constexpr int kMaxAhead = kStages - 2;  // own stages in flight after a step's wait
  for (int s_ = 0; s_ <= kMaxAhead && s_ < KT; ++s_) issue_stage(s_);
  wait_vmcnt(min(kMaxAhead, KT - 1) * kInstPerStage);  // own share of stage 0
  pp_barrier();
  if (grp == 1) pp_barrier();  // group 1 runs one phase behind
  // One K-step.  `ahead` = own stages still allowed in flight after the wait
  // (stages kt + 2 .. min(kt + S - 1, KT - 1)) is a compile-time count, so
  // the wait is one instruction: a count computed at run time compiled into
  // a branch tree of ~20 scalar instructions per step, which cost 10% of the
  // kernel.  kFirst: the MFMAs start from an inline zero, not from acc.
  auto kstep = [&](int kt, auto ahead_c, auto first_c) {
    constexpr int kAhead = decltype(ahead_c)::value;
    constexpr bool kFirst = decltype(first_c)::value;
    read_frags(kt);
    if constexpr (kAhead == kMaxAhead) issue_stage(kt + kStages - 1);
    PRICHS_WAIT_VMCNT(kAhead * kInstPerStage);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): own LDS reads done
    pp_barrier();
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        acc[i][j] = mfma_bf16(F.w[j], F.a[i], kFirst ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[i][j]);
    pp_barrier();
  };
  // Step kt allows min(S - 2, KT - 2 - kt) stages in flight (at least 0):
  // step 0 and the steady state issue stage kt + S - 1 and allow S - 2, the
  // last steps count down to 0.
  using AMax = std::integral_constant<int, kMaxAhead>;
  using A0 = std::integral_constant<int, 0>;
  if (KT - 2 >= kMaxAhead) {
    kstep(0, AMax{}, bool_c<true>{});
  } else {
    static_for(std::make_integer_sequence<int, kMaxAhead>{}, [&](auto i_c) {
      constexpr int a = kMaxAhead - 1 - decltype(i_c)::value;
      if (max(KT - 2, 0) == a) kstep(0, std::integral_constant<int, a>{}, bool_c<true>{});
    });
  }
  int kt = 1;
  for (; kt + kStages - 1 < KT; ++kt) kstep(kt, AMax{}, bool_c<false>{});
  static_for(std::make_integer_sequence<int, kMaxAhead>{}, [&](auto i_c) {
    constexpr int a = kMaxAhead - 1 - decltype(i_c)::value;
    if (kt + a + 1 < KT) kstep(kt++, std::integral_constant<int, a>{}, bool_c<false>{});
  });
  if (kt < KT) kstep(kt++, A0{}, bool_c<false>{});
  if (grp == 0) pp_barrier();  // both groups leave after the same barrier count

  // Epilogue: acc[i][j][r] = C[row m0 + wm*WM + 16i + (lane & 15)]
  //                           [packed col n0 + wn*WN + 16j + 4*(lane >> 4) + r].
  const int lr = m0 + wm * WM + fr;
  const int cq = 4 * (lane >> 4);
  if (!GATEUP && (stage_c || DSW)) {
    // Staged (down / dense): each lane's 8-byte pieces go to a row-major
    // copy of the tile in LDS, then the workgroup writes whole rows with
    // 16-byte lanes (a wave store covers 8 full 128-byte lines instead of
    // 32-byte pieces of 16 rows).  C is 16-byte aligned and ldc, n_store
    // are multiples of 8.
    constexpr int kS = Cf::kStgStride;
    lds_barrier();  // every wave is done reading the ring
    const int tcol = wn * WN + cq;
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      bf16_t *srow = lds + (wm * WM + fr + 16 * i) * kS + tcol;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const f32x4 a = acc[i][j];
        *reinterpret_cast<u32x2 *>(srow + 16 * j) =
            u32x2{pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3])};
      }
    }
    lds_barrier();
    constexpr int kChunksRow = BN / 8;  // 16-byte chunks per tile row
    if constexpr (DSW) {
      // SwiGLU backward on the staged (bf16-rounded) dA: chunk ch of row r
      // is activation columns col .. col + 7, whose gate and up
      // pre-activations are 8 contiguous values each at packed column
      // (col / kIl) 2 kIl + col % kIl and kIl on.  Each thread's chunks go in
      // batches of 8, all loads of a batch before its in-place stores;
      // chunks outside the group's rows or past Np_gu / 2 load from the
      // buffer's start and store nothing.
      constexpr int kIl = Cf::kIl;
      constexpr int kIters = BM * kChunksRow / Cf::kThreads;
      constexpr int kBatch = kIters < 8 ? kIters : 8;
      static_assert(BM * kChunksRow % Cf::kThreads == 0 && kIters % kBatch == 0,
                    "whole batches of chunks per thread");
      const int half_np = ldc / 2;
#pragma unroll 1
      for (int b0 = 0; b0 < kIters; b0 += kBatch) {
        u32x4 gv[kBatch], uv[kBatch], av[kBatch];
        bf16_t *gp[kBatch];
        int col[kBatch];
#pragma unroll
        for (int e = 0; e < kBatch; ++e) {
          const int c = tid + (b0 + e) * Cf::kThreads;
          const int r = c / kChunksRow, ch = c - r * kChunksRow;
          const int m = m0 + r;
          col[e] = n0 + 8 * ch;
          const bool ok = m < mg && col[e] < half_np;
          gp[e] = ok ? P + (long long)(row0 + m) * ldc + (col[e] / kIl) * 2 * kIl + col[e] % kIl
                     : nullptr;
          const bf16_t *src = ok ? gp[e] : P;
          gv[e] = *reinterpret_cast<const u32x4 *>(src);
          uv[e] = *reinterpret_cast<const u32x4 *>(src + kIl);
          av[e] = *reinterpret_cast<const u32x4 *>(lds + r * kS + 8 * ch);
        }
#pragma unroll
        for (int e = 0; e < kBatch; ++e) {
          if (gp[e] == nullptr) continue;
          u32x4 dgv = {0u, 0u, 0u, 0u}, duv = {0u, 0u, 0u, 0u};
          if (col[e] < n_store) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              float dg[2], du[2];
#pragma unroll
              for (int h = 0; h < 2; ++h) {
                const uint32_t gb = h ? gv[e][i] & 0xffff0000u : gv[e][i] << 16;
                const uint32_t ub = h ? uv[e][i] & 0xffff0000u : uv[e][i] << 16;
                const uint32_t ab = h ? av[e][i] & 0xffff0000u : av[e][i] << 16;
                swiglu_bwd_elem(__builtin_bit_cast(float, gb), __builtin_bit_cast(float, ub),
                                __builtin_bit_cast(float, ab), dg[h], du[h]);
              }
              dgv[i] = pack_bf16x2(dg[0], dg[1]);
              duv[i] = pack_bf16x2(du[0], du[1]);
            }
          }
          *reinterpret_cast<u32x4 *>(gp[e]) = dgv;
          *reinterpret_cast<u32x4 *>(gp[e] + kIl) = duv;
        }
      }
      return;
    }
#pragma unroll 4
    for (int c = tid; c < BM * kChunksRow; c += Cf::kThreads) {
      const int r = c / kChunksRow, ch = c - r * kChunksRow;
      const int m = m0 + r, col = n0 + 8 * ch;
      if (m < mg && col < n_store)
        *reinterpret_cast<u32x4 *>(C + (long long)(row0 + m) * ldc + col) =
            *reinterpret_cast<const u32x4 *>(lds + r * kS + 8 * ch);
    }
    return;  // the next tile's barrier keeps the ring refill behind these reads
  }
  if constexpr (GATEUP) {
    // Packed rows [n0 + wn*WN, +WN) are WN / (2 kIl) [kIl gate | kIl up]
    // blocks: in block q, gate column c (16-column piece jj) pairs with up
    // column c, kIl / 16 pieces on.
    constexpr int kPieces = Cf::kIl / 16;  // 16-column pieces per gate (or up) half
    static_assert(kPieces == 2 && NJ % 2 == 0, "pairs of 16-column pieces");
    // Each lane holds 4 consecutive values of one row in each 16-column
    // piece.  Lanes l and l + 16 (16-lane rows 2r, 2r + 1) hold columns
    // cq .. cq + 3 and cq + 4 .. cq + 7 of the same row, so for a pair of
    // pieces one v_permlane16_swap per dword hands the even row both halves
    // of the first piece and the odd row both halves of the second: with
    // stage_c (16-byte aligned outputs) every lane writes 8 consecutive
    // columns with one 16-byte store (a wave store covers 16 rows x 64 bytes
    // instead of 16 rows x 32 bytes); otherwise 8-byte stores of its own 4.
    const bool odd = (lane >> 4) & 1;
    auto store_pair = [&](bf16_t *row_ptr, int col0, u32x2 v0, u32x2 v1, bool ok0, bool ok1) {
      // col0: the pair's first column for this lane's cq (piece 1 is 16 on).
      if (stage_c) {
        const auto sx = __builtin_amdgcn_permlane16_swap(v0[0], v1[0], false, false);
        const auto sy = __builtin_amdgcn_permlane16_swap(v0[1], v1[1], false, false);
        if (odd ? ok1 : ok0)
          *reinterpret_cast<u32x4 *>(row_ptr + col0 + (odd ? 12 : 0)) =
              u32x4{sx[0], sy[0], sx[1], sy[1]};
      } else {
        if (ok0) *reinterpret_cast<u32x2 *>(row_ptr + col0) = v0;
        if (ok1) *reinterpret_cast<u32x2 *>(row_ptr + col0 + 16) = v1;
      }
    };
    if (P != nullptr && stage_c) {
      // Training forward: the gate/up pre-activations too, [rows][Np] in
      // packed column order (the backward's SwiGLU derivative needs them),
      // through a row-major copy of the tile in LDS and written as whole
      // 512-byte rows, as the down epilogue writes its tile.  Nothing reads
      // them until the backward's dA epilogue, so the stores are
      // non-temporal: the 126 MB at config 2 leave the memory-side cache to
      // the forward's weights and activations (training forward 335.5 ->
      // 328.8 us, step -6.9 us).
      constexpr int kS = Cf::kStgStride;
      lds_barrier();  // every wave is done reading the ring
      const int tcol = wn * WN + cq;
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        bf16_t *srow = lds + (wm * WM + fr + 16 * i) * kS + tcol;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const f32x4 a = acc[i][j];
          *reinterpret_cast<u32x2 *>(srow + 16 * j) =
              u32x2{pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3])};
        }
      }
      lds_barrier();
      constexpr int kChunksRow = BN / 8;  // 16-byte chunks per tile row
#pragma unroll 4
      for (int c = tid; c < BM * kChunksRow; c += Cf::kThreads) {
        const int r = c / kChunksRow, ch = c - r * kChunksRow;
        const int m = m0 + r;
        if (m < mg)
          __builtin_nontemporal_store(
              *reinterpret_cast<const u32x4 *>(lds + r * kS + 8 * ch),
              reinterpret_cast<u32x4 *>(P + (long long)(row0 + m) * Np + n0 + 8 * ch));
      }
    } else if (P != nullptr) {
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int m = lr + 16 * i;
        bf16_t *prow = P + (long long)(row0 + m) * Np;
#pragma unroll
        for (int jp = 0; jp < NJ; jp += 2) {
          const f32x4 a = acc[i][jp], b = acc[i][jp + 1];
          store_pair(prow, n0 + wn * WN + 16 * jp + cq,
                     u32x2{pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3])},
                     u32x2{pack_bf16x2(b[0], b[1]), pack_bf16x2(b[2], b[3])}, m < mg, m < mg);
        }
      }
    }
    if (stage_c && P == nullptr) {
      // Inference: the activations through LDS, [BM][BN / 2 + 8], then whole
      // 256-byte rows (config 2: 296.3 -> 293.7 us per layer; after the
      // pre-activation copy of the training forward the extra barrier costs
      // more than it gains there).
      constexpr int kSa = BN / 2 + 8;
      lds_barrier();  // every wave is done reading the ring
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        bf16_t *srow = lds + (wm * WM + fr + 16 * i) * kSa;
#pragma unroll
        for (int q = 0; q < NJ / (2 * kPieces); ++q) {
#pragma unroll
          for (int jj = 0; jj < kPieces; ++jj) {
            const int j = 2 * kPieces * q + jj;
            float h[4];
#pragma unroll
            for (int r = 0; r < 4; ++r)
              h[r] = PRICHS_BF16_SILU(acc[i][j][r]) * acc[i][j + kPieces][r];
            *reinterpret_cast<u32x2 *>(srow + (wn * WN + 2 * Cf::kIl * q) / 2 + cq + 16 * jj) =
                u32x2{pack_bf16x2(h[0], h[1]), pack_bf16x2(h[2], h[3])};
          }
        }
      }
      lds_barrier();
      constexpr int kChunksRow = BN / 16;  // 16-byte chunks per activation row
#pragma unroll 4
      for (int c = tid; c < BM * kChunksRow; c += Cf::kThreads) {
        const int r = c / kChunksRow, ch = c - r * kChunksRow;
        const int m = m0 + r, col = n0 / 2 + 8 * ch;
        if (m < mg && col < n_store)
          *reinterpret_cast<u32x4 *>(C + (long long)(row0 + m) * ldc + col) =
              *reinterpret_cast<const u32x4 *>(lds + r * kSa + 8 * ch);
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      const int m = lr + 16 * i;
      bf16_t *crow = C + (long long)(row0 + m) * ldc;
#pragma unroll
      for (int q = 0; q < NJ / (2 * kPieces); ++q) {
        u32x2 v[kPieces];
#pragma unroll
        for (int jj = 0; jj < kPieces; ++jj) {
          const int j = 2 * kPieces * q + jj;  // gate piece; up piece is j + kPieces
          float h[4];
#pragma unroll
          for (int r = 0; r < 4; ++r)
            h[r] = PRICHS_BF16_SILU(acc[i][j][r]) * acc[i][j + kPieces][r];
          v[jj] = u32x2{pack_bf16x2(h[0], h[1]), pack_bf16x2(h[2], h[3])};
        }
        const int col0 = (n0 + wn * WN + 2 * Cf::kIl * q) / 2 + cq;
        store_pair(crow, col0, v[0], v[1], m < mg && col0 < n_store, m < mg && col0 + 16 < n_store);
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
            const f32x4 a = acc[i][j];
            *reinterpret_cast<u32x2 *>(crow + col) =
                u32x2{pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3])};
          }
        }
      }
    }
  }
}

// Persistent grouped GEMM: workgroups walk the (group, M-tile, N-tile) list
// in the XCD-aware order.  CfT is the configuration of the last partial
// round (wave quantisation): when its tiles fill at most half of the
// workgroups, each of them is computed as two half-width tiles (CfT::BN =
// Cf::BN / 2) on two workgroups, so that round takes about half as long.
// Every output element is the same MFMA chain over K either way, so the
// results are bit-identical.  CfT == Cf turns this off.
template <class Cf, class CfT, bool GATEUP, bool DSW = false>
__global__ __launch_bounds__(kBf16Threads) void bf16_gemm_kernel(
    const bf16_t *__restrict__ A, const int32_t *__restrict__ a_rows, int lda,
    const bf16_t *__restrict__ B, long long b_group_stride, int Np, int K,
    bf16_t *__restrict__ C, int ldc, int n_store, const int32_t *__restrict__ offsets,
    int G, int dense_m, int stage_c, bf16_t *__restrict__ P, A2Rows a2) {
  constexpr bool kSplit = !std::is_same<Cf, CfT>::value;
  static_assert(!kSplit || (CfT::BM == Cf::BM && 2 * CfT::BN == Cf::BN && !GATEUP),
                "tail tiles are the two column halves of a down / dense tile");
  extern __shared__ __attribute__((aligned(16))) bf16_t lds[];
  WaveTileMap tm;
  build_wave_tile_map(tm, offsets, G, Cf::BM, dense_m);

  const int n_tiles = Np / Cf::BN;
  const int m_tiles = tm.m_tiles;
  const int total = m_tiles * n_tiles;
  const int nblk = gridDim.x;
  int n_full = total, n_items = total;  // tiles computed whole; work items
  if (kSplit) {
    const int tail = total % nblk;
    if (tail > 0 && 2 * tail <= nblk) {
      n_full = total - tail;
      n_items = n_full + 2 * tail;
    }
  }
  for (int t = xcd_block_id(); t < n_items; t += nblk) {
    int mt, nt;
    if (t < n_full) {
      tile_coords(t, m_tiles, n_tiles, mt, nt);
      bf16_tile<Cf, GATEUP, DSW>(A, a_rows, lda, B, b_group_stride, Np, K, C, ldc, n_store, tm,
                                 stage_c, P, lds, mt, nt, a2);
    } else if constexpr (kSplit) {
      // Items 2u, 2u + 1 are the halves of tail tile n_full + u (consecutive
      // items run on one XCD, so both halves share the A panel in its L2).
      const int u = t - n_full;
      tile_coords(n_full + u / 2, m_tiles, n_tiles, mt, nt);
      bf16_tile<CfT, GATEUP, DSW>(A, a_rows, lda, B, b_group_stride, Np, K, C, ldc, n_store, tm,
                                  stage_c, P, lds, mt, 2 * nt + (u & 1), a2);
    }
  }
}


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
    float *__restrict__ C, int ldc, int n_store, const int32_t *__restrict__ offsets, int G,
    int dense_m, float *__restrict__ P) {
  extern __shared__ float ldsf[];
  __shared__ TileMap tm;
  build_tile_map(tm, offsets, G, BM, dense_m);

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
    const int row0 = tm.offs[g];
    const int mg = tm.offs[g + 1] - row0;
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
    if (GATEUP && P != nullptr) {
      // Training forward: the pre-activations, [rows][Np] in packed order.
      const int pbase = n0 + wn * WN + (lane & 15);
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int lr = rbase + i * 16 + r;
          if (lr < mg) {
            float *prow = P + (long long)(row0 + lr) * Np + pbase;
#pragma unroll
            for (int j = 0; j < NJ; ++j) prow[j * 16] = acc[i][j][r];
          }
        }
    }
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

// ------------------------------------------------------------------------
// Skinny grouped GEMM for decode-sized groups (at most kSkinnyRows rows per
// group per M-tile).  With a handful of rows per expert there is no weight
// reuse to stage through LDS: the launch is bound by streaming the touched
// experts' packed weights from HBM once.  One workgroup of 4 waves covers
// (group, 64 packed weight rows, 32 token rows); each wave streams its own 16
// packed rows (K-contiguous, 16 bytes per lane per K-step) straight into MFMA
// operand registers, with kSkU K-steps per chunk double-buffered in registers,
// and reads the activation fragments of the (at most 32) rows from the cache.
// MFMA operands as in the tiled kernel: weights are operand A (row n = lane &
// 15, k = 8 * (lane >> 4)), activations operand B, so lane (m = lane & 15)
// ends with output columns 4 * (lane >> 4) + r, r = 0..3.
// ------------------------------------------------------------------------
namespace skinny {
constexpr int kThreads = 256;
constexpr int BM = 32;           // token rows per M-tile (two 16-row MFMA tiles)
constexpr int BN = 64;           // packed weight rows per workgroup (16 per wave)
constexpr int kSkinnyRows = 64;  // engine uses this path when every group has <= this many rows

// The wave's weight fragments of K-steps s0 .. s0+U-1 (1 KiB apart in the
// fragment-major packing).
template <int U>
__device__ inline void load_w(const bf16_t *__restrict__ wp, int s0, bf16x8 (&w)[U]) {
#pragma unroll
  for (int u = 0; u < U; ++u) w[u] = *reinterpret_cast<const bf16x8 *>(wp + (s0 + u) * 512);
}

// GATEUP: C = act [rows][ldc], packed rows [64s, 64s + 64) are one [32 gate |
// 32 up] block (the packing interleave), so N-waves 0/1 (gate) pair with
// N-waves 2/3 (up) lane for lane.  Otherwise C = y [rows][ldc].  The workgroup
// is 4 x SK waves: N-wave wn = wave & 3 covers packed rows 16 wn.., K-slice
// ks = wave >> 2 covers K [ks K/SK, (ks+1) K/SK) (more waves, so more weight
// bytes in flight per CU); slice partial sums are added in slice order.
// Activations go through LDS: per chunk of U K-steps, the 4 waves of a slice
// load its [32 rows][32 U] tile once (16 bytes per load) into one of two
// buffers, and every N-wave reads its MFMA fragments from there.
// (K / SK) % (32 * U) == 0.
// One skinny launch.  Group g owns rows [offsets[g], offsets[g+1]) of the
// row space, or with dense_T > 0 rows [g dense_T, (g+1) dense_T) whose A rows
// are 0 .. dense_T - 1 (every token of every group; offsets is not read).  A
// row r of the row space is A[a_rows[r]] when a_rows is set.  a_copy (may be
// null): the workgroups of N-slab 0 also write the A rows they stage to
// a_copy [row][lda] at their row-space rows.
struct SkinnyArgs {
  const bf16_t *A;
  const int32_t *a_rows;
  int lda;
  const bf16_t *B;
  long long b_stride;
  int K;
  bf16_t *C;
  int ldc, n_store;
  const int32_t *offsets;
  int dense_T;
  bf16_t *P;
  int ldp;
  bf16_t *a_copy;
};

// The workgroup (N-slab bx, group g, M-tile bz) of a skinny launch.
template <bool GATEUP, int U, int SK>
__device__ __forceinline__ void skinny_body(const SkinnyArgs &sa, int bx, int g, int bz) {
  const bf16_t *__restrict__ A = sa.A;
  const int32_t *__restrict__ a_rows = sa.a_rows;
  const int lda = sa.lda, K = sa.K, ldc = sa.ldc, n_store = sa.n_store, ldp = sa.ldp;
  const bf16_t *__restrict__ B = sa.B;
  const long long b_stride = sa.b_stride;
  bf16_t *__restrict__ C = sa.C;
  bf16_t *__restrict__ P = sa.P;
  constexpr int kRow = 32 * U + 8;                 // LDS row (16-byte pad: conflict-free reads)
  constexpr int kSegs = BM * 4 * U;                // 16-byte segments of one chunk tile
  constexpr int kSegPerThread = kSegs / kThreads;  // U / 2
  static_assert(kSegs % kThreads == 0, "whole segments per thread");
  __shared__ __attribute__((aligned(16))) bf16_t a_s[SK][2][BM * kRow];
  __shared__ f32x4 red_s[SK > 1 ? SK - 1 : 1][4][2][64];  // [slice-1][N-wave][tile][lane]
  __shared__ f32x4 gate_s[2][2][64];                      // [gate wave][tile][lane]
  const bool dense = sa.dense_T > 0;
  const int g0 = dense ? g * sa.dense_T : sa.offsets[g];
  const int r1 = dense ? g0 + sa.dense_T : sa.offsets[g + 1];
  const int m0 = g0 + bz * BM;
  if (m0 >= r1) return;  // uniform: this M-tile of the group is empty
  const int mrows = min(BM, r1 - m0);
  const bool two = mrows > 16;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wn = wave & 3, ks = wave >> 2;
  const int st = threadIdx.x & (kThreads - 1);  // thread within the slice
  const int Ks = K / SK;
  const int nc = Ks / (32 * U);
  // Fragment (16-row block nb, K-step ks * Ks / 32 + s) of the packed weights.
  const int nb = bx * (BN / 16) + wn;
  const bf16_t *wp =
      B + g * b_stride + ((long long)nb * (K / 32) + ks * (Ks / 32)) * 512 + lane * 8;

  // Activation staging: segment i = st + kThreads * j is (row i / (4U), 16-byte
  // column i % (4U)) of the chunk tile; rows past the group re-read its last
  // row (their outputs are never stored).
  const bf16_t *asrc[kSegPerThread];
  int adst[kSegPerThread];
  bf16_t *acpy[kSegPerThread];  // row-space copy of the staged rows (N-slab 0 only)
#pragma unroll
  for (int j = 0; j < kSegPerThread; ++j) {
    const int i = st + kThreads * j;
    const int r = i / (4 * U), sc = i % (4 * U);
    int src = min(m0 + r, r1 - 1);
    if (a_rows != nullptr)
      src = a_rows[src];
    else if (dense)
      src -= g0;
    asrc[j] = A + (long long)src * lda + ks * Ks + sc * 8;
    adst[j] = r * kRow + sc * 8;
    acpy[j] = (sa.a_copy != nullptr && bx == 0 && m0 + r < r1)
                  ? sa.a_copy + (long long)(m0 + r) * lda + ks * Ks + sc * 8
                  : nullptr;
  }
  bf16x8 areg[kSegPerThread];
  auto load_a = [&](int c) {
#pragma unroll
    for (int j = 0; j < kSegPerThread; ++j)
      areg[j] = *reinterpret_cast<const bf16x8 *>(asrc[j] + c * 32 * U);
  };
  // Chunk c's staged A values go to LDS buffer buf (and to the copy).
  auto store_a = [&](int buf, int c) {
#pragma unroll
    for (int j = 0; j < kSegPerThread; ++j) {
      *reinterpret_cast<bf16x8 *>(&a_s[ks][buf][adst[j]]) = areg[j];
      if (acpy[j] != nullptr) *reinterpret_cast<bf16x8 *>(acpy[j] + c * 32 * U) = areg[j];
    }
  };
  const int rd = (lane & 15) * kRow + 8 * (lane >> 4);  // fragment read offset, tile 0
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  auto mma = [&](const bf16x8(&w)[U], int buf) {
    const bf16_t *as = &a_s[ks][buf][rd];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      acc0 = mfma_bf16(w[u], *reinterpret_cast<const bf16x8 *>(as + 32 * u), acc0);
      if (two) acc1 = mfma_bf16(w[u], *reinterpret_cast<const bf16x8 *>(as + 16 * kRow + 32 * u), acc1);
    }
  };

  // Chunk c: A(c) is stored to buffer c & 1 during iteration c - 1; W(c) sits
  // in w0 (c even) or w1 (c odd).  Loads of chunk c + 2 are issued in
  // iteration c, A before W, unconditionally (clamped to the last chunk), so
  // the compiler's waits count exactly the loads issued after each one's.
  bf16x8 w0[U], w1[U];
  load_a(0);
  load_w<U>(wp, 0, w0);
  store_a(0, 0);
  load_a(min(1, nc - 1));
  load_w<U>(wp, min(1, nc - 1) * U, w1);
  __syncthreads();
  for (int c = 0; c < nc; c += 2) {
    mma(w0, 0);
    if (c + 1 < nc) store_a(1, c + 1);
    load_a(min(c + 2, nc - 1));
    load_w<U>(wp, min(c + 2, nc - 1) * U, w0);
    __syncthreads();
    if (c + 1 < nc) {
      mma(w1, 1);
      if (c + 2 < nc) store_a(0, c + 2);
    }
    load_a(min(c + 3, nc - 1));
    load_w<U>(wp, min(c + 3, nc - 1) * U, w1);
    __syncthreads();
  }

  if (SK > 1) {
    if (ks > 0) {
      red_s[ks - 1][wn][0][lane] = acc0;
      red_s[ks - 1][wn][1][lane] = acc1;
    }
    __syncthreads();
    if (ks == 0) {
#pragma unroll
      for (int j = 0; j < SK - 1; ++j) {
        acc0 += red_s[j][wn][0][lane];
        acc1 += red_s[j][wn][1][lane];
      }
    }
  }

  const int cq = 4 * (lane >> 4);
  const int mr = m0 + (lane & 15);
  if constexpr (GATEUP) {
    if (P != nullptr && ks == 0) {
      // Training forward: this wave's pre-activations (packed rows 16 wn..).
      const int pcol = bx * BN + wn * 16 + cq;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int m = mr + 16 * t;
        if (m < r1) {
          const f32x4 v = t == 0 ? acc0 : acc1;
          *reinterpret_cast<u32x2 *>(P + (long long)m * ldp + pcol) =
              u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        }
      }
    }
    if (ks == 0 && wn < 2) {
      gate_s[wn][0][lane] = acc0;
      gate_s[wn][1][lane] = acc1;
    }
    __syncthreads();
    if (ks == 0 && wn >= 2) {
      const int col = bx * (BN / 2) + (wn - 2) * 16 + cq;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int m = mr + 16 * t;
        if (m < r1 && col < n_store) {
          const f32x4 gv = gate_s[wn - 2][t][lane];
          const f32x4 uv = t == 0 ? acc0 : acc1;
          float h[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) h[r] = PRICHS_BF16_SILU(gv[r]) * uv[r];
          *reinterpret_cast<u32x2 *>(C + (long long)m * ldc + col) =
              u32x2{pack_bf16x2(h[0], h[1]), pack_bf16x2(h[2], h[3])};
        }
      }
    }
  } else if (ks == 0) {
    const int col = bx * BN + wn * 16 + cq;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int m = mr + 16 * t;
      if (m < r1 && col < n_store) {
        const f32x4 v = t == 0 ? acc0 : acc1;
        *reinterpret_cast<u32x2 *>(C + (long long)m * ldc + col) =
            u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
      }
    }
  }
}
template <bool GATEUP, int U, int SK>
__global__ __launch_bounds__(kThreads * SK) void skinny_gemm_kernel(SkinnyArgs sa) {
  skinny_body<GATEUP, U, SK>(sa, (int)blockIdx.x, (int)blockIdx.y, (int)blockIdx.z);
}

// The router workgroup's arguments in the decode launch (router_quad_body).
struct RouterArgs {
  const bf16_t *x;
  const float *w, *bias, *concept;
  int n_concept, T, d, E, k;
  float *logits;
  int32_t *topk_idx;
  float *topk_w;
  int32_t *block_counts;
  rq::FusedPerm perm;
  const float *w_lds;
};

// Decode launch: workgroup 0 routes the batch (one router workgroup covers
// it) and writes its permutation; workgroups 1.. are the dense gate/up GEMM
// (N-slab, group, M-tile) = the workgroups of skinny_gemm_kernel<true, U, 1>
// over nx x ny x .. blocks, dispatched after the router's so it starts first.
template <int U>
__global__ __launch_bounds__(kThreads) void decode_gate_up_router_kernel(SkinnyArgs sa,
                                                                        RouterArgs ra, int nx,
                                                                        int ny) {
  static_assert(kThreads == rq::kRouterThreads, "one workgroup size for both roles");
  extern __shared__ __attribute__((aligned(16))) float router_wt_s[];  // W^T [8][d + 4]
  const int b = (int)blockIdx.x;
  if (b == 0) {
    rq::router_quad_body<bf16_t>(ra.x, ra.w, ra.bias, ra.concept, ra.n_concept, ra.T, ra.d, ra.E,
                                 ra.k, ra.logits, ra.topk_idx, ra.topk_w, ra.block_counts,
                                 ra.perm, ra.w_lds, 0, router_wt_s);
    return;
  }
  const int i = b - 1;
  skinny_body<true, U, 1>(sa, i % nx, (i / nx) % ny, i / (nx * ny));
}
}  // namespace skinny

size_t il_of(int dtype) { return dtype == PRICHS_DTYPE_BF16 ? (size_t)Bf16::kIl : (size_t)fp::kIl; }
size_t bn_of(int dtype) { return dtype == PRICHS_DTYPE_BF16 ? (size_t)Bf16::BN : (size_t)fp::BN; }

int check_gemm_shape(size_t d, size_t f, int dtype, const char *who) {
  if (!dtype_ok(dtype)) return fail(PRICHS_ERR_INVALID_ARGUMENT, "%s: bad dtype %d", who, dtype);
  const size_t q = dtype == PRICHS_DTYPE_BF16 ? (size_t)kBf16KMultiple : (size_t)fp::BK;
  if (d == 0 || f == 0 || d % q || f % q)
    return fail(PRICHS_ERR_UNSUPPORTED, "%s: d=%zu and f=%zu must be positive multiples of %zu",
                who, d, f, q);
  if (d > (1u << 20) || f > (1u << 20))
    return fail(PRICHS_ERR_UNSUPPORTED, "%s: d=%zu or f=%zu too large", who, d, f);
  // The kernels address one group's packed weights with 32-bit element
  // offsets: [Np, d] gate/up (Np <= 2 roundup(f, 32) + 256) and [roundup(d,
  // 256), f] down must stay below 2^32 elements.
  if ((2 * roundup(f, 32) + 256) * d > (size_t)UINT32_MAX || roundup(d, 256) * f > (size_t)UINT32_MAX)
    return fail(PRICHS_ERR_UNSUPPORTED, "%s: packed weights of d=%zu, f=%zu exceed 2^32 elements",
                who, d, f);
  return PRICHS_OK;
}

template <typename T> void put(void *out, size_t i, float v);
template <> void put<float>(void *out, size_t i, float v) { static_cast<float *>(out)[i] = v; }
template <> void put<bf16_t>(void *out, size_t i, float v) {
  static_cast<bf16_t *>(out)[i] = f32_to_bf16(v);
}

// Element (n, k) of a packed [Np, K] weight.  f32: row-major.  bf16:
// fragment-major, the operand layout of v_mfma_f32_16x16x32_bf16: fragment
// (n / 16, k / 32) is 1 KiB contiguous, lane l = n % 16 + 16 * ((k % 32) / 8)
// holding k % 8 = 0..7 in 16 bytes, fragments of one 16-row block ordered by k.
// A wave instruction then moves one whole fragment (one contiguous KiB), to
// LDS in the tiled kernel and straight into registers in the skinny one.
inline size_t packed_index(size_t n, size_t k, size_t K, bool bf16) {
  if (!bf16) return n * K + k;
  const size_t lane = (n & 15) + 16 * ((k & 31) >> 3);
  return (((n >> 4) * (K >> 5) + (k >> 5)) * 64 + lane) * 8 + (k & 7);
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
    for (size_t k = 0; k < d; ++k)
      put<T>(out, packed_index(p, k, d, sizeof(T) == 2), col < f ? src[k * f + col] : 0.0f);
  }
}

template <typename T> void pack_down_impl(const float *down, size_t d, size_t f, void *out) {
  const size_t np = roundup(d, kPadRowsDown);
  for (size_t n = 0; n < np; ++n)
    for (size_t k = 0; k < f; ++k)
      put<T>(out, packed_index(n, k, f, sizeof(T) == 2), n < d ? down[k * d + n] : 0.0f);
}

// Workgroups of the persistent bf16 launches: one per CU, or at most
// PRICHS_GEMM_MAX_CUS (read once) -- a cap that leaves CUs to other work
// and measures how the kernels scale with the number of CUs in use.
int gemm_cu_limit(int cus) {
  static const int cap = [] {
    const char *v = std::getenv("PRICHS_GEMM_MAX_CUS");
    const int n = v ? std::atoi(v) : 0;
    return n > 0 ? n : 0;
  }();
  return cap > 0 && cap < cus ? cap : cus;
}

// Half-width configuration of the last partial round (down / dense only,
// and only where half a tile is still a whole number of B loads per wave).
template <class Cf, bool GATEUP>
using TailCfg = typename std::conditional<
    GATEUP || (Cf::BN / 2) % (Cf::kRowsPerInst * Cf::kWaves) != 0, Cf,
    Bf16Cfg<Cf::BM, Cf::BN / 2, Cf::WGM, Cf::WGN, Cf::kStages>>::type;

// Persistent grid of a bf16 launch: one workgroup per CU (the LDS ring allows
// one), fewer when the launch has fewer tiles (twice the tiles when the last
// round may be split into halves).
template <class Cf, bool GATEUP>
size_t bf16_grid(size_t max_rows, int G, int Np, int cus) {
  const bool halves = !std::is_same<Cf, TailCfg<Cf, GATEUP>>::value;
  const size_t ub = (max_rows / Cf::BM + G) * (size_t)(Np / Cf::BN) * (halves ? 2 : 1);
  return std::max<size_t>(1, std::min<size_t>(ub, (size_t)gemm_cu_limit(cus)));
}

template <class Cf, bool GATEUP, bool DSW = false>
int launch_bf16(const void *A, const int32_t *a_rows, int lda, const void *B, long long b_stride,
                int Np, int K, void *Cp, int ldc, int n_store, const int32_t *offsets, int G,
                int dense_m, size_t max_rows, int cus, hipStream_t s, void *pre,
                A2Rows a2 = A2Rows()) {
  using CfT = TailCfg<Cf, GATEUP>;
  const int grid = (int)bf16_grid<Cf, GATEUP>(max_rows, G, Np, cus);
  static bool attr_set = false;
  if (!attr_set) {
    PRICHS_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void *>(&bf16_gemm_kernel<Cf, CfT, GATEUP, DSW>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)Cf::kLdsBytes),
                   "grouped gemm: set LDS size");
    attr_set = true;
  }
  // 16-byte epilogue stores (down / dense: rows staged in LDS; gate/up:
  // lane pairs' halves exchanged) need C (and the pre-activations) 16-byte
  // aligned and whole 8-column chunks; otherwise each lane stores its 8-byte
  // pieces directly.
  const int stage_c = (GATEUP || PRICHS_GEMM_STAGE_C) &&
                      reinterpret_cast<uintptr_t>(Cp) % 16 == 0 && ldc % 8 == 0 &&
                      n_store % 8 == 0 && reinterpret_cast<uintptr_t>(pre) % 16 == 0;
  static_assert(CfT::kLdsBytes <= Cf::kLdsBytes, "tail tiles fit the launch's LDS");
  if (DSW && !stage_c)
    return fail(PRICHS_ERR_UNSUPPORTED,
                "grouped gemm: the SwiGLU-backward epilogue needs 16-byte aligned pre-activations");
  hipLaunchKernelGGL((bf16_gemm_kernel<Cf, CfT, GATEUP, DSW>), dim3(grid), dim3(Cf::kThreads), Cf::kLdsBytes, s,
                     static_cast<const bf16_t *>(A), a_rows, lda, static_cast<const bf16_t *>(B),
                     b_stride, Np, K, static_cast<bf16_t *>(Cp), ldc, n_store, offsets, G, dense_m,
                     stage_c, static_cast<bf16_t *>(pre), a2);
  PRICHS_LAUNCH_CHECK("grouped gemm launch");
  return PRICHS_OK;
}

// Tile-times (in units of the configuration's own tile) of a persistent
// launch of `tiles` tiles on `grid` workgroups: whole rounds, plus the last
// partial round -- 0.6 of a tile-time when its tiles are split into
// half-width tiles (split allowed and twice the tail fits the grid; measured
// on MI355X: 8192 x 2304 x 1536 takes 1.59 tile-times of a full round), else
// a full one.
double launch_tile_times(size_t tiles, size_t grid, bool split) {
  const size_t full = tiles / grid, tail = tiles % grid;
  if (tail == 0) return (double)full;
  return (double)full + (split && 2 * tail <= grid ? 0.6 : 1.0);
}

// Work of one 128 x 384 tile against a 256 x 256 one, and the rate of the
// narrower tile (fewer MFMAs per barrier and per byte staged) against the
// square one's, measured on MI355X in whole rounds (32768 x 1536 x 1536:
// 124.7 us as 1024 wide tiles, 120.2 us as 768 square ones).  A 256 x 288
// tile is 1.125 square tiles of work at the square tile's rate per flop.
constexpr double kWideWork = 0.75, kWideRate = 0.96, kTallWork = 1.125;

// Tile shape of a dense launch of M rows and Np packed columns: the one with
// the fewest estimated square-tile-times on the grid launch_bf16 gives it
// (0: 256 x 256 with half-width tails, 1: 128 x 384, 2: 256 x 288).
int dense_tile_choice(size_t M, size_t Np, int cus) {
  const size_t sq = ((M + Bf16Down::BM - 1) / Bf16Down::BM) * (Np / Bf16Down::BN);
  double best = launch_tile_times(sq, bf16_grid<Bf16Down, false>(M, 1, Np, cus), true);
  int choice = 0;
  if (Np % Bf16Wide::BN == 0) {
    const size_t wd = ((M + Bf16Wide::BM - 1) / Bf16Wide::BM) * (Np / Bf16Wide::BN);
    const double t = launch_tile_times(wd, bf16_grid<Bf16Wide, false>(M, 1, Np, cus), false) *
                     kWideWork / kWideRate;
    if (t < best) best = t, choice = 1;
  }
  if (Np % Bf16Tall::BN == 0) {
    const size_t tl = ((M + Bf16Tall::BM - 1) / Bf16Tall::BM) * (Np / Bf16Tall::BN);
    const double t =
        launch_tile_times(tl, bf16_grid<Bf16Tall, false>(M, 1, Np, cus), false) * kTallWork;
    if (t < best) best = t, choice = 2;
  }
  return choice;
}

template <bool GATEUP, int U, int SK>
int launch_skinny_u(const void *A, const int32_t *a_rows, int lda, const void *B,
                    long long b_stride, int Np, int K, void *Cp, int ldc, int n_store,
                    const int32_t *offsets, int G, int mtiles, hipStream_t s, void *pre,
                    void *a_copy = nullptr) {
  static_assert(Bf16::kIl == skinny::BN / 2, "a skinny slab is one [gate | up] block");
  const skinny::SkinnyArgs sa{static_cast<const bf16_t *>(A), a_rows, lda,
                              static_cast<const bf16_t *>(B), b_stride, K,
                              static_cast<bf16_t *>(Cp), ldc, n_store, offsets, 0,
                              static_cast<bf16_t *>(pre), Np, static_cast<bf16_t *>(a_copy)};
  hipLaunchKernelGGL((skinny::skinny_gemm_kernel<GATEUP, U, SK>),
                     dim3(Np / skinny::BN, G, mtiles), dim3(skinny::kThreads * SK), 0, s, sa);
  PRICHS_LAUNCH_CHECK("skinny grouped gemm launch");
  return PRICHS_OK;
}

// K split SK <= PRICHS_SKINNY_SK and K-steps per chunk U <= PRICHS_SKINNY_U,
// each the largest that divides K evenly (every slice a whole number of
// chunks; K is a multiple of 64).  Combinations whose LDS would exceed
// ~70 KB (U = 8 with SK = 4) are not instantiated.  Measured at the decode
// shape (T = 32, d = 1536, f = 1280): SK = 1, U = 4 is fastest (gate/up 17.0
// us vs 18-23 us for SK = 2 or 4 and U = 2 or 8).
#ifndef PRICHS_SKINNY_SK
#define PRICHS_SKINNY_SK 1
#endif
#ifndef PRICHS_SKINNY_U
#define PRICHS_SKINNY_U 4
#endif
template <bool GATEUP>
int launch_skinny(const void *A, const int32_t *a_rows, int lda, const void *B, long long b_stride,
                  int Np, int K, void *Cp, int ldc, int n_store, const int32_t *offsets, int G,
                  size_t max_group_rows, hipStream_t s, void *pre, void *a_copy = nullptr) {
  const int mtiles = (int)std::max<size_t>(1, (max_group_rows + skinny::BM - 1) / skinny::BM);
  int sk = PRICHS_SKINNY_SK;
  while (sk > 1 && K % (sk * 64) != 0) sk /= 2;
  int u = PRICHS_SKINNY_U;
  while (u > 2 && (K / sk) % (32 * u) != 0) u /= 2;
  if (u == 8 && sk == 4) u = 4;
#define PRICHS_SKINNY(U_, SK_)                                                                   \
  if (u == U_ && sk == SK_)                                                                     \
  return launch_skinny_u<GATEUP, U_, SK_>(A, a_rows, lda, B, b_stride, Np, K, Cp, ldc, n_store, \
                                          offsets, G, mtiles, s, pre, a_copy)
  PRICHS_SKINNY(2, 1);
  PRICHS_SKINNY(4, 1);
  PRICHS_SKINNY(8, 1);
  PRICHS_SKINNY(2, 2);
  PRICHS_SKINNY(4, 2);
  PRICHS_SKINNY(8, 2);
  PRICHS_SKINNY(2, 4);
  PRICHS_SKINNY(4, 4);
#undef PRICHS_SKINNY
  return fail(PRICHS_ERR_UNSUPPORTED, "skinny gemm: no kernel for K=%d", K);
}

// max_group_rows bounds every group's row count (offsets[g+1] - offsets[g]);
// bf16 launches whose groups all fit the skinny kernel's reach take it.
// pre (gate/up only, may be null): the pre-activations [rows][Np], packed order.
int launch_grouped(bool gateup, const void *A, const int32_t *a_rows, int lda, const void *B,
                   long long b_stride, int Np, int K, void *Cp, int ldc, int n_store,
                   const int32_t *offsets, int G, int dense_m, size_t max_rows, int dtype,
                   hipStream_t s, size_t max_group_rows, void *pre = nullptr) {
  if (dtype == PRICHS_DTYPE_BF16 && dense_m == 0 && max_group_rows <= (size_t)skinny::kSkinnyRows &&
      K % kBf16KMultiple == 0 && Np % skinny::BN == 0) {
    return gateup ? launch_skinny<true>(A, a_rows, lda, B, b_stride, Np, K, Cp, ldc, n_store,
                                        offsets, G, max_group_rows, s, pre)
                  : launch_skinny<false>(A, a_rows, lda, B, b_stride, Np, K, Cp, ldc, n_store,
                                         offsets, G, max_group_rows, s, nullptr);
  }
  const int cus = device_cu_count();
  if (cus <= 0) return fail(PRICHS_ERR_HIP, "grouped gemm: cannot query the device");
  if (dtype == PRICHS_DTYPE_BF16) {
    if (gateup)
      return launch_bf16<Bf16, true>(A, a_rows, lda, B, b_stride, Np, K, Cp, ldc, n_store,
                                     offsets, G, dense_m, max_rows, cus, s, pre);
    const int shape = offsets == nullptr ? dense_tile_choice((size_t)dense_m, (size_t)Np, cus) : 0;
    if (shape == 1)
      return launch_bf16<Bf16Wide, false>(A, a_rows, lda, B, b_stride, Np, K, Cp, ldc, n_store,
                                          offsets, G, dense_m, max_rows, cus, s, nullptr);
    if (shape == 2)
      return launch_bf16<Bf16Tall, false>(A, a_rows, lda, B, b_stride, Np, K, Cp, ldc, n_store,
                                          offsets, G, dense_m, max_rows, cus, s, nullptr);
    return launch_bf16<Bf16Down, false>(A, a_rows, lda, B, b_stride, Np, K, Cp, ldc, n_store,
                                        offsets, G, dense_m, max_rows, cus, s, nullptr);
  } else {
    const size_t ub = (max_rows / fp::BM + G) * (size_t)(Np / fp::BN);
    const int grid = (int)std::max<size_t>(1, std::min<size_t>(ub, (size_t)cus * 4));
    auto kern = gateup ? fp::grouped_gemm_kernel<true> : fp::grouped_gemm_kernel<false>;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(fp::kThreads), fp::kLdsBytes, s,
                       static_cast<const float *>(A), a_rows, lda,
                       static_cast<const float *>(B), b_stride, Np, K,
                       static_cast<float *>(Cp), ldc, n_store, offsets, G, dense_m,
                       gateup ? static_cast<float *>(pre) : nullptr);
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

namespace prichs {
int grouped_gate_up_swiglu_rows(const void *x, const int32_t *row_token, const int32_t *offsets,
                                size_t G, size_t max_rows, size_t max_group_rows,
                                const void *w_packed, size_t d, size_t f, int dtype, void *act,
                                void *stream, void *pre) {
  if (int rc = check_gemm_shape(d, f, dtype, "gate_up")) return rc;
  PRICHS_REQUIRE(G >= 1 && G <= (size_t)kMaxGroups, "gate_up: G=%zu outside [1, %d]", G,
                 kMaxGroups);
  PRICHS_REQUIRE(x && row_token && offsets && w_packed && act, "gate_up: null pointer argument");
  PRICHS_REQUIRE(max_rows <= (size_t)INT32_MAX, "gate_up: max_rows too large");
  const size_t np = gate_up_np(f, dtype);
  PRICHS_REQUIRE(pre == nullptr || max_rows * np <= (size_t)INT64_MAX / 4,
                 "gate_up: pre-activation buffer too large");
  return launch_grouped(true, x, row_token, (int)d, w_packed, (long long)(np * d), (int)np,
                        (int)d, act, (int)f, (int)f, offsets, (int)G, 0, max_rows, dtype,
                        as_stream(stream), std::min(max_rows, max_group_rows), pre);
}

int grouped_down_rows(const void *act, const int32_t *offsets, size_t G, size_t max_rows,
                      size_t max_group_rows, const void *w_packed, size_t d, size_t f, int dtype,
                      void *y, void *stream) {
  if (int rc = check_gemm_shape(d, f, dtype, "down")) return rc;
  PRICHS_REQUIRE(G >= 1 && G <= (size_t)kMaxGroups, "down: G=%zu outside [1, %d]", G,
                 kMaxGroups);
  PRICHS_REQUIRE(act && offsets && w_packed && y, "down: null pointer argument");
  PRICHS_REQUIRE(max_rows <= (size_t)INT32_MAX, "down: max_rows too large");
  const size_t np = roundup(d, kPadRowsDown);
  return launch_grouped(false, act, nullptr, (int)f, w_packed, (long long)(np * f), (int)np,
                        (int)f, y, (int)d, (int)d, offsets, (int)G, 0, max_rows, dtype,
                        as_stream(stream), std::min(max_rows, max_group_rows));
}
bool decode_dense_applies(size_t T, size_t d, size_t f, size_t E, size_t k, size_t n_shared,
                          int dtype, const void *x, const float *w_router) {
  constexpr size_t kTokens = rq::kRouterThreads / 8;  // one quad-router workgroup
  return dtype == PRICHS_DTYPE_BF16 && n_shared == 1 && E > 4 && E <= 8 && k >= 1 && k <= E &&
         T >= 1 && T <= kTokens && d % 128 == 0 && (size_t)8 * (d + 4) * 4 <= 150 * 1024 &&
         f % kBf16KMultiple == 0 && d <= (1u << 20) && f <= (1u << 20) &&
         reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(w_router) % 16 == 0;
}

int decode_gate_up_router(const void *x, size_t T, size_t d, size_t f, size_t E, size_t k,
                          const float *w_router, const float *w_lds, const float *router_bias,
                          const float *concept_bias, size_t n_concept, float *logits,
                          int32_t *topk_idx, float *topk_w, int32_t *block_counts,
                          int32_t *offsets, int32_t *row_token, float *row_weight,
                          int32_t *token_row, int32_t *dense_row, const void *w_gate_up,
                          void *act_dense, void *stream) {
  PRICHS_REQUIRE(decode_dense_applies(T, d, f, E, k, 1, PRICHS_DTYPE_BF16, x, w_router),
                 "decode_gate_up_router: T=%zu, d=%zu, f=%zu, E=%zu, k=%zu not a decode shape",
                 T, d, f, E, k);
  PRICHS_REQUIRE(x && w_router && router_bias && logits && topk_idx && topk_w && block_counts &&
                     offsets && row_token && row_weight && token_row && dense_row && w_gate_up &&
                     act_dense,
                 "decode_gate_up_router: null pointer argument");
  PRICHS_REQUIRE(concept_bias != nullptr || n_concept == 0,
                 "decode_gate_up_router: concept_bias is NULL but n_concept=%zu", n_concept);
  constexpr int U = 4;
  const size_t np = gate_up_np(f, PRICHS_DTYPE_BF16);
  const int G = (int)E + 1;
  const int nx = (int)(np / skinny::BN);
  const int mtiles = (int)((T + skinny::BM - 1) / skinny::BM);
  const size_t lds = (size_t)8 * (d + 4) * sizeof(float);
  static int attr_bytes = 0;
  if ((int)lds > attr_bytes) {
    PRICHS_HIP_TRY(hipFuncSetAttribute(
                       reinterpret_cast<const void *>(&skinny::decode_gate_up_router_kernel<U>),
                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                   "decode_gate_up_router: set LDS size");
    attr_bytes = (int)lds;
  }
  const skinny::SkinnyArgs sa{static_cast<const bf16_t *>(x), nullptr, (int)d,
                              static_cast<const bf16_t *>(w_gate_up), (long long)(np * d), (int)d,
                              static_cast<bf16_t *>(act_dense), (int)f, (int)f, nullptr, (int)T,
                              nullptr, (int)np, nullptr};
  const int nc = (int)(n_concept < E ? n_concept : E);
  const skinny::RouterArgs ra{static_cast<const bf16_t *>(x), w_router, router_bias, concept_bias,
                              nc, (int)T, (int)d, (int)E, (int)k, logits, topk_idx, topk_w,
                              block_counts,
                              rq::FusedPerm{offsets, row_token, row_weight, token_row, dense_row},
                              w_lds};
  const unsigned grid = 1u + (unsigned)(nx * G * mtiles);
  hipLaunchKernelGGL((skinny::decode_gate_up_router_kernel<U>), dim3(grid), dim3(skinny::kThreads),
                     lds, as_stream(stream), sa, ra, nx, G);
  PRICHS_LAUNCH_CHECK("decode gate/up + router launch");
  return PRICHS_OK;
}

int decode_down(const void *act_dense, const int32_t *dense_row, const int32_t *offsets, size_t T,
                size_t d, size_t f, size_t E, size_t k, const void *w_down, void *y, void *act,
                void *stream) {
  if (int rc = check_gemm_shape(d, f, PRICHS_DTYPE_BF16, "decode_down")) return rc;
  PRICHS_REQUIRE(act_dense && dense_row && offsets && w_down && y && act,
                 "decode_down: null pointer argument");
  PRICHS_REQUIRE(T >= 1 && T <= (size_t)skinny::kSkinnyRows && k <= E,
                 "decode_down: T=%zu, k=%zu, E=%zu not a decode shape", T, k, E);
  const size_t np = roundup(d, kPadRowsDown);
  return launch_skinny<false>(act_dense, dense_row, (int)f, w_down, (long long)(np * f), (int)np,
                              (int)f, y, (int)d, (int)d, offsets, (int)E + 1, T,
                              as_stream(stream), nullptr, act);
}

int grouped_gemm_rows(const void *A, const int32_t *a_rows, size_t lda, const void *B,
                      size_t b_group_stride, size_t Np, size_t K, void *C, size_t ldc,
                      size_t n_store, const int32_t *offsets, size_t G, size_t max_rows,
                      size_t max_group_rows, int dtype, void *stream) {
  if (int rc = check_gemm_shape(Np, K, dtype, "grouped gemm")) return rc;
  PRICHS_REQUIRE(Np % bn_of(dtype) == 0,
                 "grouped gemm: Np=%zu is not a whole number of weight tiles", Np);
  PRICHS_REQUIRE(G >= 1 && G <= (size_t)kMaxGroups, "grouped gemm: G=%zu outside [1, %d]", G,
                 kMaxGroups);
  PRICHS_REQUIRE(A && offsets && B && C, "grouped gemm: null pointer argument");
  PRICHS_REQUIRE(lda >= K && ldc >= n_store && n_store <= Np && lda % 8 == 0 && ldc % 4 == 0,
                 "grouped gemm: lda=%zu, ldc=%zu, n_store=%zu invalid for K=%zu, Np=%zu", lda,
                 ldc, n_store, K, Np);
  PRICHS_REQUIRE(max_rows <= (size_t)INT32_MAX && lda <= (size_t)INT32_MAX &&
                     ldc <= (size_t)INT32_MAX && b_group_stride * G <= (size_t)INT64_MAX,
                 "grouped gemm: operands too large");
  return launch_grouped(false, A, a_rows, (int)lda, B, (long long)b_group_stride, (int)Np,
                        (int)K, C, (int)ldc, (int)n_store, offsets, (int)G, 0, max_rows, dtype,
                        as_stream(stream), std::min(max_rows, max_group_rows));
}

bool dact_swiglu_bwd_fusable(size_t d, size_t np_f, const void *gu, size_t np, size_t f,
                             size_t max_rows, size_t max_group_rows, int dtype) {
  // The tiled kernel's shapes (launch_grouped takes the skinny kernel for
  // decode-sized groups), 16-byte aligned pre-activations of whole 8-column
  // chunks, and a packed width whose activation columns the N-tiles cover.
  const size_t mg = std::min(max_rows, max_group_rows);
  const bool skinny = mg <= (size_t)skinny::kSkinnyRows && d % kBf16KMultiple == 0 &&
                      np_f % skinny::BN == 0;
  return dtype == PRICHS_DTYPE_BF16 && !skinny && reinterpret_cast<uintptr_t>(gu) % 16 == 0 &&
         np % 8 == 0 && f % 8 == 0 && np / 2 <= np_f && np_f % Bf16Down::BN == 0 &&
         max_rows <= (size_t)INT32_MAX && d <= (size_t)INT32_MAX && np <= (size_t)INT32_MAX;
}

int grouped_dact_swiglu_bwd(const void *dy, size_t d, const void *w_down_t, size_t b_group_stride,
                            size_t np_f, void *gu, size_t np, size_t f, const int32_t *offsets,
                            size_t G, size_t max_rows, size_t max_group_rows, int dtype,
                            void *stream, bool *fused, const void *a2, size_t a2_g,
                            size_t a2_row0) {
  *fused = false;
  if (int rc = check_gemm_shape(np_f, d, dtype, "dA + SwiGLU backward")) return rc;
  PRICHS_REQUIRE(dy && w_down_t && gu && offsets && G >= 1 && G <= (size_t)kMaxGroups,
                 "dA + SwiGLU backward: null pointer or G=%zu", G);
  if (!dact_swiglu_bwd_fusable(d, np_f, gu, np, f, max_rows, max_group_rows, dtype))
    return PRICHS_OK;
  const int cus = device_cu_count();
  if (cus <= 0) return fail(PRICHS_ERR_HIP, "dA + SwiGLU backward: cannot query the device");
  A2Rows alt;
  if (a2 != nullptr) {
    // Element distance from dy to a2 (both bf16, so exact).
    alt.delta = (long long)(reinterpret_cast<intptr_t>(a2) - reinterpret_cast<intptr_t>(dy)) / 2;
    alt.g = (int)a2_g;
    alt.row0 = (int)a2_row0;
  }
  *fused = true;
  return launch_bf16<Bf16Down, false, true>(dy, nullptr, (int)d, w_down_t,
                                            (long long)b_group_stride, (int)np_f, (int)d, nullptr,
                                            (int)np, (int)f, offsets, (int)G, 0, max_rows, cus,
                                            as_stream(stream), gu, alt);
}
}  // namespace prichs

// A group can hold all max_rows rows, so the public entry points take that as
// the per-group bound.
extern "C" int prichs_grouped_gate_up_swiglu(const void *x, const int32_t *row_token,
                                             const int32_t *offsets, size_t G, size_t max_rows,
                                             const void *w_packed, size_t d, size_t f, int dtype,
                                             void *act, void *stream) {
  return grouped_gate_up_swiglu_rows(x, row_token, offsets, G, max_rows, max_rows, w_packed, d,
                                     f, dtype, act, stream, nullptr);
}

extern "C" int prichs_grouped_down(const void *act, const int32_t *offsets, size_t G,
                                   size_t max_rows, const void *w_packed, size_t d, size_t f,
                                   int dtype, void *y, void *stream) {
  return grouped_down_rows(act, offsets, G, max_rows, max_rows, w_packed, d, f, dtype, y, stream);
}

extern "C" size_t prichs_packed_weight_elems(size_t K, size_t N, int dtype) {
  if (!dtype_ok(dtype)) return 0;
  return roundup(N, kPadRowsDown) * K;
}

extern "C" int prichs_pack_weight(const float *w, size_t K, size_t N, int dtype,
                                  void *packed_out) {
  // The layout of a packed down projection: [roundup(N, 256)][K] = W^T.
  if (int rc = check_gemm_shape(N, K, dtype, "pack_weight")) return rc;
  PRICHS_REQUIRE(w && packed_out, "pack_weight: null pointer argument");
  if (dtype == PRICHS_DTYPE_BF16)
    pack_down_impl<bf16_t>(w, N, K, packed_out);
  else
    pack_down_impl<float>(w, N, K, packed_out);
  return PRICHS_OK;
}

extern "C" int prichs_gemm(const void *a, size_t lda, size_t M, size_t K, const void *w_packed,
                           size_t N, void *c, size_t ldc, int dtype, void *stream) {
  if (int rc = check_gemm_shape(N, K, dtype, "gemm")) return rc;
  PRICHS_REQUIRE(lda >= K && ldc >= N, "gemm: lda=%zu < K=%zu or ldc=%zu < N=%zu", lda, K, ldc, N);
  PRICHS_REQUIRE(M <= (size_t)INT32_MAX && lda <= (size_t)INT32_MAX && ldc <= (size_t)INT32_MAX,
                 "gemm: M=%zu or leading dimensions too large", M);
  PRICHS_REQUIRE(lda % 8 == 0 && ldc % 4 == 0, "gemm: lda must be a multiple of 8, ldc of 4");
  if (M == 0) return PRICHS_OK;
  PRICHS_REQUIRE(a && w_packed && c, "gemm: null pointer argument");
  const size_t np = roundup(N, kPadRowsDown);
  return launch_grouped(false, a, nullptr, (int)lda, w_packed, (long long)(np * K), (int)np,
                        (int)K, c, (int)ldc, (int)N, nullptr, 1, (int)M, M, dtype,
                        as_stream(stream), M);
}
