// backward.hip -- kernels of the MoE layer backward (the engine drives them).
//
// Replaces the reference's training-step MoE backward: GpuModelEngine::
// gpu_moe_init_backward / gpu_moe_backward_expert / gpu_moe_backward_shared /
// gpu_moe_backward_router (crates/prichs-cuda/src/engine.rs:2242-2789), their
// kernels (crates/prichs-cuda/src/kernels.cu:455-480 SwiGLU backward, 926-991
// gather / router dot / scatter) and the host router VJP
// moe_router_unbiased_backward (crates/prichs-core/src/backward.rs:269-287),
// as driven by Model::train_step (crates/prichs-model/src/model.rs:1474-1561).
// The reference runs one expert at a time with host round trips; here every
// stage covers all groups (routed experts and the shared expert) in one launch
// over the engine's row space, and nothing is summed with atomics, so the
// result is deterministic.
//
// Kernels here:
//   rows_kernel       dY[r] = w_r * d_out[t_r], xg[r] = x[t_r], and the router
//                     scalar s_r = <y[r], d_out[t_r]> (routed rows);
//   swiglu_bwd_kernel dG, dU from dA and the gate/up pre-activations, in place
//                     in the packed [gate 32 | up 32] column order;
//   wgrad kernels     dW[group] += A_g^T B_g over each group's rows (MFMA);
//   combine_kernel    the router VJP and the input gradient of each token;
//   router wgrad      dW_router += x^T d_logits as per-expert weighted sums of
//                     the gathered rows (two deterministic passes).
#include <algorithm>

#include "common.hpp"

namespace prichs {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kIl = 32;  // packed gate/up interleave of both dtypes: [32 gate | 32 up] blocks

// ------------------------------------------------------ 8-element vectors --
template <typename T> struct V8;
template <> struct V8<float> {
  __device__ static void load(const float *p, float v[8]) {
    const float4 a = *reinterpret_cast<const float4 *>(p);
    const float4 b = *reinterpret_cast<const float4 *>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
  __device__ static void load_nt(const float *p, float v[8]) {
    typedef float f4_t __attribute__((ext_vector_type(4)));
    const f4_t a = __builtin_nontemporal_load(reinterpret_cast<const f4_t *>(p));
    const f4_t b = __builtin_nontemporal_load(reinterpret_cast<const f4_t *>(p + 4));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = a[i];
      v[4 + i] = b[i];
    }
  }
  __device__ static void store(float *p, const float v[8]) {
    *reinterpret_cast<float4 *>(p) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4 *>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
  }
  __device__ static void copy(const float *src, float *dst) {
    *reinterpret_cast<float4 *>(dst) = *reinterpret_cast<const float4 *>(src);
    *reinterpret_cast<float4 *>(dst + 4) = *reinterpret_cast<const float4 *>(src + 4);
  }
};
template <> struct V8<bf16_t> {
  __device__ static void load(const bf16_t *p, float v[8]) {
    const u32x4 u = *reinterpret_cast<const u32x4 *>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __builtin_bit_cast(float, u[i] << 16);
      v[2 * i + 1] = __builtin_bit_cast(float, u[i] & 0xffff0000u);
    }
  }
  // Non-temporal (streaming) load, for data read for the last time.
  __device__ static void load_nt(const bf16_t *p, float v[8]) {
    const u32x4 u = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __builtin_bit_cast(float, u[i] << 16);
      v[2 * i + 1] = __builtin_bit_cast(float, u[i] & 0xffff0000u);
    }
  }
  __device__ static void store(bf16_t *p, const float v[8]) {
    u32x4 u;
#pragma unroll
    for (int i = 0; i < 4; ++i) u[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
    *reinterpret_cast<u32x4 *>(p) = u;
  }
  __device__ static void copy(const bf16_t *src, bf16_t *dst) {
    *reinterpret_cast<u32x4 *>(dst) = *reinterpret_cast<const u32x4 *>(src);
  }
};

// Sum over the 64 lanes of a wave in a fixed butterfly order (every lane
// ends with the same bits).
__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = v + __shfl_xor(v, m, 64);
  return v;
}

// ------------------------------------------------------------- rows pass --
// One wave per token t, over its k routed rows r_s = token_row[t k + s]
// (and, with `shared`, its shared row T k + t): dY[r] = w_r * d_out[t]
// (kernels.cu:926-944; w = 1 on the shared row, whose gradient the reference
// feeds straight to the shared expert, engine.rs:2513-2703), xg[r] = x[t]
// (the gathered expert input of the weight gradients), and for routed rows
// s_r = sum_c y[r][c] * d_out[t][c] (kernels.cu:946-969: the dot of the
// unweighted expert output with the layer's output gradient), each lane
// summing its columns in order and the wave by a fixed butterfly.  d_out[t]
// and x[t] are read once for all of the token's rows.
template <typename T, int KC>
__global__ __launch_bounds__(256) void rows_kernel(const T *__restrict__ x,
                                                   const T *__restrict__ d_out,
                                                   const T *__restrict__ y,
                                                   const int32_t *__restrict__ token_row,
                                                   const float *__restrict__ row_weight, int T_,
                                                   int k_rt, int d, int shared, T *__restrict__ dy,
                                                   T *__restrict__ xg, float *__restrict__ scal) {
#pragma clang fp contract(off)
  constexpr int kMax = KC > 0 ? KC : PRICHS_MAX_TOPK;
  const int k = KC > 0 ? KC : k_rt;
  const int lane = threadIdx.x & 63;
  const int t = __builtin_amdgcn_readfirstlane((int)(blockIdx.x * 4 + (threadIdx.x >> 6)));
  if (t >= T_) return;
  int rr[kMax];
  float w[kMax], sacc[kMax];
#pragma unroll
  for (int sl = 0; sl < kMax; ++sl) {
    rr[sl] = sl < k ? token_row[(size_t)t * k + sl] : 0;
    w[sl] = sl < k ? row_weight[rr[sl]] : 0.f;
    sacc[sl] = 0.f;
  }
  const size_t rsh = (size_t)T_ * k + t;  // the shared row
  const T *go = d_out + (size_t)t * d;
  const T *xr = x + (size_t)t * d;
  // x[t] is copied as raw bits (8 elements: 16 bytes in bf16, 32 in f32).
  using XRaw = typename std::conditional<sizeof(T) == 2, u32x4, u32x4[2]>::type;
  for (int c = lane * 8; c < d; c += 64 * 8) {
    float g[8];
    V8<T>::load(go + c, g);
    XRaw xv;
    __builtin_memcpy(&xv, xr + c, sizeof(XRaw));
#pragma unroll
    for (int sl = 0; sl < kMax; ++sl) {
      if (sl < k) {
        float o[8], yv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = w[sl] * g[j];
        V8<T>::store(dy + (size_t)rr[sl] * d + c, o);
        __builtin_memcpy(xg + (size_t)rr[sl] * d + c, &xv, sizeof(XRaw));
        V8<T>::load(y + (size_t)rr[sl] * d + c, yv);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float p = yv[j] * g[j];
          sacc[sl] = sacc[sl] + p;
        }
      }
    }
    if (shared) {
      V8<T>::store(dy + rsh * d + c, g);
      __builtin_memcpy(xg + rsh * d + c, &xv, sizeof(XRaw));
    }
  }
#pragma unroll
  for (int sl = 0; sl < kMax; ++sl) {
    if (sl < k) {
      const float sr = wave_sum(sacc[sl]);
      if (lane == 0) scal[rr[sl]] = sr;
    }
  }
}

// ------------------------------------------------------ SwiGLU backward --
// kernels.cu:459-480 per element (swiglu_bwd_elem).  gu holds
// the packed pre-activations [rows, np] (block q: gate columns 32q.. at
// 64q.., up at 64q + 32..) and receives dG, dU in the same places; padding
// blocks (columns >= f) are cleared so the dX product sees zeros there.
template <typename T>
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(T *__restrict__ gu,
                                                         const T *__restrict__ da, int rows,
                                                         int f, int np) {
#pragma clang fp contract(off)
  const int per_row = np / (2 * kIl) * (kIl / 8);  // 8-column chunks of gate per row
  const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (long long)rows * per_row) return;
  const int r = (int)(gid / per_row);
  const int rem = (int)(gid - (long long)r * per_row);
  const int q = rem / (kIl / 8), h = rem - q * (kIl / 8);
  const int col = q * kIl + h * 8;
  T *gp = gu + (size_t)r * np + (size_t)q * 2 * kIl + h * 8;
  T *up = gp + kIl;
  float g[8], u[8], a[8], dg[8], du[8];
  if (col >= f) {
#pragma unroll
    for (int j = 0; j < 8; ++j) dg[j] = 0.f;
    V8<T>::store(gp, dg);
    V8<T>::store(up, dg);
    return;
  }
  V8<T>::load(gp, g);
  V8<T>::load(up, u);
  V8<T>::load(da + (size_t)r * f + col, a);
#pragma unroll
  for (int j = 0; j < 8; ++j) swiglu_bwd_elem(g[j], u[j], a[j], dg[j], du[j]);
  V8<T>::store(gp, dg);
  V8<T>::store(up, du);
}

// ------------------------------------------------------ weight gradients --
// dW[group g] = beta dW + A_g^T B_g, A_g = rows [offsets[g], offsets[g+1]) of
// A [*, lda] (columns 0..P), B_g the same rows of B [*, ldb] (columns 0..Q):
// the reference's cuBLAS sgemm calls, beta = 1 (engine.rs:2345-2362 for
// dW_down, 2417-2451 for dW_gate / dW_up; 2619-2654 for the shared expert);
// beta = 0 is the same after zero_grads (engine.rs:710-720), whose gradients
// of experts without rows are zero.  Groups are the engine's: routed
// experts 0..E-1 then the shared expert (group E); group g's matrices sit at
// slot g + 1 (routed) or 0 (shared) of the caller's gradients, slot s at
// out + s * slot_stride.
//   plain:  out0[i][j] (ldo) for i < P, j < Q.
//   gateup: B's columns are packed gate/up (block q = [32 gate | 32 up]); column
//           p goes to out0 (gate) or out1 (up) at column 32 (p / 64) + p % 32
//           when that is < f.
// Workgroups: one per (group, 128 x 128 output tile), the shared group's
// tiles first (it has the most rows).  Workgroups are dealt round-robin to
// the 8 XCDs, so block b runs on XCD b % 8; each XCD takes a contiguous band
// of every group's tiles (tiles in a band share A and B panels in that XCD's
// L2), and every group's tiles spread over all XCDs.
namespace wg {
constexpr int BP = 128, BQ = 128;
constexpr int kThreads = 256;
}  // namespace wg

__device__ __forceinline__ int slot_of(int g, int E) { return g < E ? g + 1 : 0; }

// Block -> (group, tile), or false past the last tile (the grid is
// 8 * band * G with band = ceil(tiles / 8)).
__device__ __forceinline__ bool wgrad_item(int G, int tiles, int &g, int &tile) {
  const int band = (tiles + 7) / 8;
  const int xcd = (int)(blockIdx.x & 7), s = (int)(blockIdx.x >> 3);
  const int gi = s / band;
  tile = xcd * band + (s - gi * band);
  g = (gi + G - 1) % G;  // the last group (shared) first
  return gi < G && tile < tiles;
}

// Output element pointer of (i, j) or nullptr when outside the gradient.
template <bool GATEUP>
__device__ __forceinline__ float *wgrad_dst(float *out0, float *out1, int ldo, long long base,
                                            int i, int j, int P, int Q, int f) {
  if (i >= P || j >= Q) return nullptr;
  if (!GATEUP) return out0 + base + (long long)i * ldo + j;
  const int q = j / (2 * kIl), w = j - q * 2 * kIl;
  const int col = q * kIl + (w & (kIl - 1));
  if (col >= f) return nullptr;
  return (w < kIl ? out0 : out1) + base + (long long)i * ldo + col;
}

// --- bf16: v_mfma_f32_16x16x32_bf16, both operands read transposed from LDS.
// 256 x 256 output tiles, 8 waves as 2 (P) x 4 (Q) of 128 x 64 each; a K-step
// is 32 rows.  Both 32 x 256 operand tiles go from global memory to LDS with
// buffer_load ... lds (16 bytes per lane, no VGPR round trip) into a ring of 4
// stages, 3 ahead of the MFMAs; rows past the chunk's end load as zeros (their
// offsets are past the buffer's range).  Tile rows are 512 bytes of 32 chunks,
// chunk c of row R stored at c ^ ((2R) & 15).  ds_read_b64_tr_b16 hands lane i
// of a 16-lane group column i of the 4 rows x 16 columns the group addresses,
// so lane 16g + m, reading row 4g + m/4 (and 16 rows on) at columns
// 4(m % 4).., receives the 8 K values {4g..4g+3, 16+4g..16+4g+3} of one
// column: the same K slots for both operands.
//
// Balance: a group of m > kSplitRows rows (the shared expert, a hot expert)
// is split over K into n = ceil(m / kSplitRows) chunks of equal length
// (a multiple of 32), so work items are of similar size.  Chunk c of a split
// group stores its tile to partial slot (the group's first slot) + c, and
// wgrad_reduce_kernel then adds the chunk sum, in chunk order, to the
// gradient: dW + (((p0 + p1) + p2) + ...), one addition to dW like an
// unsplit group's.  Deterministic, no atomics and no waiting between
// workgroups.
namespace wgb {
constexpr int BP = 256, BQ = 256, BK = 32;
constexpr int kThreads = 512;
constexpr int kRowBytes = 2 * BP;                     // one tile row: 256 bf16
constexpr uint32_t kTileBytes = BK * kRowBytes;       // 16 KiB: one operand tile
constexpr uint32_t kStageBytes = 2 * kTileBytes;      // A tile then B tile
constexpr int kStages = 4;
constexpr size_t kLdsBytes = (size_t)kStages * kStageBytes;  // 128 KiB
constexpr uint32_t kHiOff = 16 * kRowBytes;           // rows 16.. of a tile
constexpr uint32_t kOutOfRange = 0x80000000u;         // buffer offset that loads zeros
constexpr int kSplitRows = 2560;
static_assert(BQ == 4 * 64 && BP == 2 * 128, "wave grid 2 x 4 of 128 x 64");
static_assert(kThreads == 8 * 64, "ping-pong K loop: two groups of 4 waves, one of each per SIMD");
}  // namespace wgb

// Chunking of a group of m > 0 rows: nc chunks of L rows (the last shorter).
__device__ __forceinline__ void wg_split(int m, int &L, int &nc) {
  const int s = (m + wgb::kSplitRows - 1) / wgb::kSplitRows;
  L = ((m + s - 1) / s + 31) / 32 * 32;
  nc = (m + L - 1) / L;
}

__device__ __forceinline__ int wg_key(int row) { return (2 * row) & 15; }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t wg_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                           0x00020000);
}
__device__ __forceinline__ void wg_dma(__amdgpu_buffer_rsrc_t r, uint32_t voff, bf16_t *lds_dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      r, (__attribute__((address_space(3))) void *)lds_dst, 16, voff, 0, 0, 0);
}
// ds_read_b64_tr_b16 with an immediate byte offset, as inline asm (the
// builtin makes the compiler wait for every LDS DMA in flight); the result is
// pending until wg_wait_tied() takes it.
template <int OFF>
__device__ __forceinline__ u32x2 wg_read_tr(uint32_t lds_byte_addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset is 16 bits");
  u32x2 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(lds_byte_addr), "n"(OFF));
  return r;
}
__device__ __forceinline__ void wg_wait_tied(u32x2 (&a)[8]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]),
                 "+v"(a[6]), "+v"(a[7])
               :
               : "memory");
}
// s_waitcnt with only vmcnt constrained (gfx9 encoding, vmcnt < 16 here).
#define PRICHS_WG_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (15 << 8))

// One work item: P rows [i0, i0 + BPT) x Q columns [j0, j0 + 256) of group g's
// dW over the item's rows (BPT = 256: a whole tile; 128: half of one).
template <bool GATEUP, int BPT>
__device__ __forceinline__ void wgrad_item(
    const bf16_t *__restrict__ A, int lda, uint32_t a_bytes, const bf16_t *__restrict__ B,
    int ldb, uint32_t b_bytes, int E, int P, int Q, float *out0, float *out1, int ldo,
    long long slot_stride, int f, float *__restrict__ part, int beta, bf16_t *lds, int g,
    int a_row_lo, int b_row_lo, int mg, int pslot, int i0, int j0) {
  using namespace wgb;
  static_assert(BPT == 256 || BPT == 128, "whole or half tiles");
  // A tile: [BK][BPT] bf16 (rows of kRowA bytes); B tile: [BK][256].
  constexpr int kRowA = 2 * BPT;
  constexpr uint32_t kTileA = BK * kRowA;
  constexpr uint32_t kStage = kTileA + kTileBytes;
  constexpr uint32_t kHiA = 16 * kRowA;
  constexpr int kIB = BPT / 2 / 16;           // 16-row A blocks per wave
  constexpr int kInstA = BPT == 256 ? 2 : 1;  // A DMA instructions per wave and stage
  constexpr int kInst = kInstA + 2;           // with B's two

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int wp = wave >> 2, wq = wave & 3;
  const __amdgpu_buffer_rsrc_t ra = wg_rsrc(A, a_bytes), rb = wg_rsrc(B, b_bytes);

  // DMA (B, 512-byte rows): wave w's instruction i fills tile rows 4w + 2i,
  // + 1; lane l lands in row 4w + 2i + l/32, physical chunk l % 32, holding
  // logical chunk (l % 32) ^ key(row).  A (kRowA-byte rows) likewise: whole
  // tiles as B; half tiles one instruction of rows 4w .. 4w + 3, lane l in
  // row 4w + l/16, physical chunk l % 16.
  uint32_t a_col[kInstA], b_col[2];
  int a_row[kInstA], b_row[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int R = 4 * wave + 2 * i + (lane >> 5);
    const int lc = (lane & 31) ^ wg_key(R);
    b_row[i] = R;
    b_col[i] = 2u * (uint32_t)(j0 + lc * 8);
  }
#pragma unroll
  for (int i = 0; i < kInstA; ++i) {
    const int R = BPT == 256 ? 4 * wave + 2 * i + (lane >> 5) : 4 * wave + (lane >> 4);
    const int lc = (BPT == 256 ? (lane & 31) : (lane & 15)) ^ wg_key(R);
    a_row[i] = R;
    a_col[i] = 2u * (uint32_t)(i0 + lc * 8);
  }
  auto issue = [&](int kt) {
    bf16_t *sa = lds + (size_t)(kt & (kStages - 1)) * (kStage / 2);
    bf16_t *sb = sa + kTileA / 2;
#pragma unroll
    for (int i = 0; i < kInstA; ++i) {
      const int rr = kt * BK + a_row[i];
      const bool ok = rr < mg;
      const uint32_t row = (uint32_t)(a_row_lo + rr);
      wg_dma(ra, ok ? row * (uint32_t)lda * 2u + a_col[i] : kOutOfRange,
             sa + (BPT == 256 ? 4 * wave + 2 * i : 4 * wave) * BPT);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int rr = kt * BK + b_row[i];
      const bool ok = rr < mg;
      const uint32_t row = (uint32_t)(b_row_lo + rr);
      wg_dma(rb, ok ? row * (uint32_t)ldb * 2u + b_col[i] : kOutOfRange,
             sb + (4 * wave + 2 * i) * BQ);
    }
  };

  // Transposing reads: lane 16g + m reads row 4g + m/4 at column
  // 16 blk + 4 (m % 4) of the wave's columns (BPT / 2 of A, 64 of B).
  const uint32_t lds_base = (uint32_t)(size_t)(const __attribute__((address_space(3))) bf16_t *)lds;
  uint32_t a_rd[kIB], b_rd[4];
  {
    const int g4 = lane >> 4, m = lane & 15;
    const int R = 4 * g4 + (m >> 2);
#pragma unroll
    for (int blk = 0; blk < kIB; ++blk) {
      const int ca = wp * (BPT / 2) + blk * 16 + 4 * (m & 3);
      a_rd[blk] = lds_base + (uint32_t)(R * kRowA + (((ca >> 3) ^ wg_key(R)) << 4) + (ca & 7) * 2);
    }
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      const int cb = wq * 64 + blk * 16 + 4 * (m & 3);
      b_rd[blk] = lds_base + kTileA +
                  (uint32_t)(R * kRowBytes + (((cb >> 3) ^ wg_key(R)) << 4) + (cb & 7) * 2);
    }
  }

  f32x4 acc[4][kIB];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < kIB; ++i) acc[j][i] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int KT = (mg + BK - 1) / BK;
  // Ping-pong K loop (as the forward GEMM's): waves 0-3 (group 0) and 4-7
  // (group 1) sit one per SIMD each.  Every wave runs, per K-step kt, a
  // memory phase (the transposing reads of stage kt, its share of stage
  // kt + 3, a wait for its share of stage kt + 1 and for its reads), a
  // barrier, an MFMA phase, a barrier; group 1 runs one barrier behind, so on
  // each SIMD one wave multiplies while the other reads and loads.
  //  - Stage s is first read after b(2s-1); both groups waited for their
  //    shares of it in their memory phases of step s - 1, which end at
  //    b(2s-2) and b(2s-1).
  //  - Stage kt + 3 goes to stage kt - 1's slot; both groups' reads of stage
  //    kt - 1 completed before b(2kt-2) and b(2kt-1), and step kt's memory
  //    phases start after b(2kt-1) and b(2kt).
  // Each output element is the same MFMA chain over K, so the results do not
  // depend on the schedule.
  const int grp = wave >> 2;
  auto pp_barrier = [] {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };
  issue(0);
  if (KT > 1) issue(1);
  if (KT > 2) issue(2);
  // Own share of stage 0 (kInst instructions per stage and wave).
  if (KT > 2)
    PRICHS_WG_VMCNT(2 * kInst);
  else if (KT > 1)
    PRICHS_WG_VMCNT(kInst);
  else
    PRICHS_WG_VMCNT(0);
  pp_barrier();
  if (grp == 1) pp_barrier();  // group 1 runs one phase behind
  // One K-step; kAhead = this wave's stages still allowed in flight after the
  // wait (stages kt + 2 .. min(kt + 3, KT - 1)), a compile-time count.
  auto kstep = [&](int kt, auto ahead_c) {
    constexpr int kAhead = decltype(ahead_c)::value;
    const uint32_t st = (uint32_t)(kt & (kStages - 1)) * kStage;
    u32x2 alo[8], ahi[8], bt[8];  // bt: B lo (0..3) and hi (4..7); A: kIB used
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      bt[blk] = wg_read_tr<0>(b_rd[blk] + st);
      bt[4 + blk] = wg_read_tr<(int)kHiOff>(b_rd[blk] + st);
    }
#pragma unroll
    for (int blk = 0; blk < 8; ++blk) {
      if (blk < kIB) {
        alo[blk] = wg_read_tr<0>(a_rd[blk] + st);
        ahi[blk] = wg_read_tr<(int)kHiA>(a_rd[blk] + st);
      } else {
        alo[blk] = ahi[blk] = u32x2{0u, 0u};
      }
    }
    if constexpr (kAhead == 2) issue(kt + 3);
    PRICHS_WG_VMCNT(kInst * kAhead);
    wg_wait_tied(bt);
    wg_wait_tied(alo);
    wg_wait_tied(ahi);
    pp_barrier();
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      const bf16x8 bf =
          __builtin_bit_cast(bf16x8, u32x4{bt[jb][0], bt[jb][1], bt[4 + jb][0], bt[4 + jb][1]});
#pragma unroll
      for (int ib = 0; ib < kIB; ++ib) {
        const bf16x8 af =
            __builtin_bit_cast(bf16x8, u32x4{alo[ib][0], alo[ib][1], ahi[ib][0], ahi[ib][1]});
        acc[jb][ib] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf, af, acc[jb][ib], 0, 0, 0);
      }
    }
    pp_barrier();
  };
  // Steps that issue stage kt + 3, then the last (up to three).
  int kt = 0;
  for (; kt + 3 < KT; ++kt) kstep(kt, std::integral_constant<int, 2>{});
  if (kt + 2 < KT) kstep(kt++, std::integral_constant<int, 1>{});
  if (kt + 1 < KT) kstep(kt++, std::integral_constant<int, 0>{});
  if (kt < KT) kstep(kt++, std::integral_constant<int, 0>{});
  if (grp == 0) pp_barrier();  // both groups leave after the same barrier count

  // acc[jb][ib] lane l holds out[i = 16 ib + l % 16][j = 16 jb + 4 (l / 16) + r]
  // of the wave's (BPT / 2) x 64 block.
  //
  // The tile leaves through the stage ring (idle after the last K-step), 128
  // rows of 1 KiB at a time: the waves holding them write their fragments to
  // LDS (float4 chunk c of row r at c ^ (r & 15), no bank conflicts either
  // way), then each wave stores 16 whole rows, one 1 KiB row per
  // instruction, instead of 16 rows x 64 bytes per instruction.
  const long long base = (long long)slot_of(g, E) * slot_stride;
  float *const pbase = pslot >= 0 ? part + (long long)pslot * P * Q : nullptr;
  const bool rmw = pslot < 0 && beta != 0;  // dW += tile (beta = 1, an unsplit group)
  f32x4 *const st = reinterpret_cast<f32x4 *>(lds);
  constexpr int kPasses = BPT / 128;
#pragma unroll
  for (int h = 0; h < kPasses; ++h) {
    if (kPasses == 1 || wp == h) {
#pragma unroll
      for (int jb = 0; jb < 4; ++jb)
#pragma unroll
        for (int ib = 0; ib < kIB; ++ib) {
          const int r = (kPasses == 1 ? wp * (BPT / 2) : 0) + ib * 16 + (lane & 15);
          const int c = wq * 16 + jb * 4 + (lane >> 4);
          st[r * 64 + (c ^ (r & 15))] = acc[jb][ib];
        }
    }
    __syncthreads();
    // Rows in batches of 8: all loads of a batch (LDS, and the old values
    // for a read-modify-write) are issued before its stores.
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      f32x4 v[8];
      float *dst[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int r = wave * 16 + b * 8 + e;
        const int i = i0 + h * 128 + r, j = j0 + 4 * lane;
        v[e] = st[r * 64 + (lane ^ (r & 15))];
        dst[e] = pbase != nullptr ? (i < P && j < Q ? pbase + (long long)i * Q + j : nullptr)
                                  : wgrad_dst<GATEUP>(out0, out1, ldo, base, i, j, P, Q, f);
      }
      if (rmw) {
        float4 old[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          old[e] = dst[e] ? *reinterpret_cast<const float4 *>(dst[e]) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          v[e][0] = old[e].x + v[e][0];
          v[e][1] = old[e].y + v[e][1];
          v[e][2] = old[e].z + v[e][2];
          v[e][3] = old[e].w + v[e][3];
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (dst[e]) {
          // The gradients go back to the caller and nothing in the step reads
          // them again: non-temporal stores keep their 211 MB (config 2) out
          // of the memory-side cache (training step -15 us).  Split-K
          // partials are read right after by the reduce pass: plain stores.
          if (pbase == nullptr)
            __builtin_nontemporal_store(v[e], reinterpret_cast<f32x4 *>(dst[e]));
          else
            *reinterpret_cast<float4 *>(dst[e]) = make_float4(v[e][0], v[e][1], v[e][2], v[e][3]);
        }
    }
    if (h + 1 < kPasses) __syncthreads();  // the next pass reuses the LDS rows
  }
}

// The tile kernel: one work item per workgroup.  Items are the groups in
// launch order (shared first), each as its chunks x tiles; when the items
// fill the last round of `cus` workgroups at most half, each of that round's
// items is computed as two half-height items (128 P rows) on two
// workgroups, so the round takes about half as long.  Every output element
// is the same MFMA chain over the item's rows either way.  HALVES selects
// this: dW_down's launch takes it (config 2: 360 items, a last round of 104
// on 256 CUs, 152 -> 144 us); dW_gate/up's does not (its last rounds are
// fuller, and with the half-height path compiled in its whole items ran
// 1-3% slower).
template <bool GATEUP, bool HALVES>
__global__ __launch_bounds__(wgb::kThreads) void wgrad_bf16_kernel(
    const bf16_t *__restrict__ A, int lda, uint32_t a_bytes, const bf16_t *__restrict__ B,
    int ldb, uint32_t b_bytes, const int32_t *__restrict__ offsets, int G, int E, int P, int Q,
    int tiles_q, int tiles, float *out0, float *out1, int ldo, long long slot_stride, int f,
    float *__restrict__ part, int beta, int cus, const bf16_t *__restrict__ A2, uint32_t a2_bytes,
    const bf16_t *__restrict__ B2, uint32_t b2_bytes, int alt_g, int alt_row0) {
  using namespace wgb;
  extern __shared__ __attribute__((aligned(16))) bf16_t lds[];
  // The offsets come to LDS in one parallel load.
  __shared__ int item[6];  // group (-1: none), first row, end row, partial slot (-1: none), tile, half
  __shared__ int offs_s[PRICHS_MAX_EXPERTS + 2];
  if ((int)threadIdx.x <= G) offs_s[threadIdx.x] = offsets[threadIdx.x];
  __syncthreads();
  if (threadIdx.x == 0) {
    int n_items = 0;
    for (int g = 0; g < G; ++g) {
      const int m = offs_s[g + 1] - offs_s[g];
      if (m <= 0) continue;
      int L, nc;
      wg_split(m, L, nc);
      n_items += nc * tiles;
    }
    const int tail = HALVES && cus > 0 ? n_items % cus : 0;
    const bool halves = tail > 0 && 2 * tail <= cus;
    const int n_whole = halves ? n_items - tail : n_items;
    // Block b runs on XCD b % 8.  The busy blocks (the grid is an upper bound)
    // are renumbered so that each XCD takes a contiguous run of them,
    // consecutive tiles that share operand panels in its L2: in each whole
    // round of `cus` blocks XCD x takes [round start + x cus/8, + cus/8), and
    // in a last partial round each XCD's run is its share of that round.
    int rest = (int)blockIdx.x, half = -1;
    const int busy = halves ? n_whole + 2 * tail : n_items;
    if (cus > 0 && cus % 8 == 0 && rest < busy) {
      const int full = busy - busy % cus;
      if (rest < full) {
        const int r0 = rest - rest % cus, p = rest % cus;
        rest = r0 + (p % 8) * (cus / 8) + p / 8;
      } else {
        const int q = rest - full, R = busy - full;
        int pre = 0;
        for (int y = 0; y < q % 8; ++y) pre += (R - y + 7) / 8;  // the blocks of XCD y
        rest = full + pre + q / 8;
      }
    }
    if (rest >= n_whole) {
      const int u = rest - n_whole;
      rest = halves && u < 2 * tail ? n_whole + u / 2 : n_items;  // n_items: no item
      half = u & 1;
    }
    int pslot = 0;
    item[0] = -1;
    for (int gi = 0; gi < G && rest < n_items; ++gi) {
      const int g = (gi + G - 1) % G;
      const int lo = offs_s[g], m = offs_s[g + 1] - lo;
      if (m <= 0) continue;
      int L, nc;
      wg_split(m, L, nc);
      if (rest < nc * tiles) {
        const int c = rest / tiles;
        item[0] = g;
        item[1] = lo + c * L;
        item[2] = min(lo + (c + 1) * L, lo + m);
        item[3] = nc == 1 ? -1 : pslot + c;
        item[4] = rest - c * tiles;
        item[5] = half;
        break;
      }
      rest -= nc * tiles;
      if (nc > 1) pslot += nc;
    }
  }
  __syncthreads();
  const int g = item[0];
  if (g < 0) return;
  const int row_lo = item[1];
  const int mg = item[2] - row_lo;
  const int pslot = item[3];
  const int tile = item[4];
  const int half = item[5];
  const int tp = tile / tiles_q;
  const int i0 = tp * BP, j0 = (tile - tp * tiles_q) * BQ;
  // Group alt_g's rows may live in other buffers: its rows alt_row0.. of the
  // row space are rows 0.. of A2 / B2 where those are given.
  const bool alt_a = g == alt_g && A2 != nullptr, alt_b = g == alt_g && B2 != nullptr;
  const bf16_t *const Ai = alt_a ? A2 : A;
  const bf16_t *const Bi = alt_b ? B2 : B;
  const uint32_t abi = alt_a ? a2_bytes : a_bytes, bbi = alt_b ? b2_bytes : b_bytes;
  const int a_row_lo = alt_a ? row_lo - alt_row0 : row_lo;
  const int b_row_lo = alt_b ? row_lo - alt_row0 : row_lo;
  if (half < 0) {
    wgrad_item<GATEUP, 256>(Ai, lda, abi, Bi, ldb, bbi, E, P, Q, out0, out1, ldo, slot_stride, f,
                            part, beta, lds, g, a_row_lo, b_row_lo, mg, pslot, i0, j0);
  } else if constexpr (HALVES) {
    wgrad_item<GATEUP, 128>(Ai, lda, abi, Bi, ldb, bbi, E, P, Q, out0, out1, ldo, slot_stride, f,
                            part, beta, lds, g, a_row_lo, b_row_lo, mg, pslot, i0 + 128 * half,
                            j0);
  }
}

// Finishes the groups the tile kernel does not write whole: a split group
// gets its partials in chunk order, dW = beta dW + (((p0 + p1) + p2) + ...);
// with beta = 0 a group without rows gets zeros.  (split = 0: the f32 kernel,
// which splits nothing.)
template <bool GATEUP>
__global__ __launch_bounds__(256) void wgrad_reduce_kernel(const float *__restrict__ part,
                                                           const int32_t *__restrict__ offsets,
                                                           int G, int E, int P, int Q, float *out0,
                                                           float *out1, int ldo,
                                                           long long slot_stride, int f, int beta,
                                                           int split) {
  __shared__ int sg[PRICHS_MAX_EXPERTS + 1], snc[PRICHS_MAX_EXPERTS + 1],
      sps[PRICHS_MAX_EXPERTS + 1];
  __shared__ int n_split;
  __shared__ int offs_s[PRICHS_MAX_EXPERTS + 2];
  if ((int)threadIdx.x <= G) offs_s[threadIdx.x] = offsets[threadIdx.x];
  __syncthreads();
  if (threadIdx.x == 0) {
    int pslot = 0, n = 0;
    for (int gi = 0; gi < G; ++gi) {
      const int g = (gi + G - 1) % G;
      const int m = offs_s[g + 1] - offs_s[g];
      if (m <= 0) {
        if (beta == 0) {  // nc = 0: written as zeros
          sg[n] = g;
          snc[n] = 0;
          sps[n] = 0;
          ++n;
        }
        continue;
      }
      if (!split) continue;
      int L, nc;
      wg_split(m, L, nc);
      if (nc > 1) {
        sg[n] = g;
        snc[n] = nc;
        sps[n] = pslot;
        ++n;
        pslot += nc;
      }
    }
    n_split = n;
  }
  __syncthreads();
  // Each group's P x Q gradient as float4 units, grid-strided, two units per
  // thread and step.  Chunk c's partial is read through a buffer resource of
  // its own; chunks past the last have an empty range and read as zeros
  // without touching memory, so every batch issues its 8 loads unconditionally
  // and the in-order sum selects which to add.  The partials are read once and
  // are dead afterwards, so the loads are non-temporal (cache policy 2): they
  // leave the caches to the operands of the kernels that follow (dW_gate/up
  // 222.7 -> 218.9 us with its reduce, training step -2.6 us; same bits).
  constexpr int kStreamingLoad = 2;
  const long long PQ = (long long)P * Q;
  const int q4n = Q / 4, n4 = P * q4n;
  const int stride = (int)gridDim.x * 256;
  for (int s = 0; s < n_split; ++s) {
    const long long gbase = (long long)slot_of(sg[s], E) * slot_stride;
    const int nc = snc[s];
    const float *p0 = part + (long long)sps[s] * PQ;
    for (int u0 = (int)(blockIdx.x * 256 + threadIdx.x); u0 < n4; u0 += 2 * stride) {
      float *dst[2];
      uint32_t off[2];
#pragma unroll
      for (int w = 0; w < 2; ++w) {
        const int u = u0 + w * stride;
        const int i = u / q4n, j = 4 * (u - i * q4n);
        dst[w] = u < n4 ? wgrad_dst<GATEUP>(out0, out1, ldo, gbase, i, j, P, Q, f) : nullptr;
        off[w] = u < n4 ? (uint32_t)(((long long)i * Q + j) * 4) : wgb::kOutOfRange;
      }
      f32x4 sum[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
      for (int c0 = 0; c0 < nc; c0 += 4) {
        f32x4 v[4][2];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const bool have = c0 + c < nc;
          const __amdgpu_buffer_rsrc_t r =
              wg_rsrc(p0 + (have ? c0 + c : 0) * PQ, have ? (uint32_t)(PQ * 4) : 0u);
#pragma unroll
          for (int w = 0; w < 2; ++w)
            v[c][w] = __builtin_bit_cast(f32x4,
                                         __builtin_amdgcn_raw_buffer_load_b128(r, off[w], 0, kStreamingLoad));
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const bool first = c0 + c == 0, use = c0 + c < nc;
#pragma unroll
          for (int w = 0; w < 2; ++w)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float a = sum[w][e] + v[c][w][e];
              sum[w][e] = first ? v[c][w][e] : use ? a : sum[w][e];
            }
        }
      }
#pragma unroll
      for (int w = 0; w < 2; ++w) {
        if (dst[w] == nullptr) continue;
        float4 r = make_float4(sum[w][0], sum[w][1], sum[w][2], sum[w][3]);
        if (beta != 0) {
          const float4 d = *reinterpret_cast<const float4 *>(dst[w]);
          r.x = d.x + r.x;
          r.y = d.y + r.y;
          r.z = d.z + r.z;
          r.w = d.w + r.w;
        }
        // The finished gradient: non-temporal, as in the tile kernel.
        __builtin_nontemporal_store(f32x4{r.x, r.y, r.z, r.w}, reinterpret_cast<f32x4 *>(dst[w]));
      }
    }
  }
}

// --- f32 (the fp32-checked mode): v_mfma_f32_16x16x4_f32, K-steps of 16 rows
// through padded LDS tiles, register double buffering.  Lane l's operand is
// element (row l / 16, column l % 16) of a 4-row slice: a plain LDS read.
namespace wgf {
constexpr int BK = 16;
constexpr int kLd = 128 + 4;  // padded LDS row (floats)
constexpr int kTile = BK * kLd;
constexpr size_t kLdsBytes = 2 * 2 * (size_t)kTile * sizeof(float);  // A and B, two buffers
}  // namespace wgf

template <bool GATEUP>
__global__ __launch_bounds__(wg::kThreads) void wgrad_f32_kernel(
    const float *__restrict__ A, int lda, const float *__restrict__ B, int ldb,
    const int32_t *__restrict__ offsets, int G, int E, int P, int Q, int tiles_q, int tiles,
    float *out0, float *out1, int ldo, long long slot_stride, int f, int beta) {
  using namespace wgf;
  extern __shared__ __attribute__((aligned(16))) float ldsw[];
  int g, tile;
  if (!wgrad_item(G, tiles, g, tile)) return;
  const int row_lo = offsets[g];
  const int mg = offsets[g + 1] - row_lo;
  if (mg <= 0) return;
  const int tp = tile / tiles_q;
  const int i0 = tp * wg::BP, j0 = (tile - tp * tiles_q) * wg::BQ;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wp = wave >> 1, wq = wave & 1;
  // Loads: thread t moves rows t / 32 and t / 32 + 8, columns 4 (t % 32)...
  const int lrow = tid >> 5, lc4 = (tid & 31) * 4;
  // Columns past P / Q read column 0 instead (their outputs are dropped).
  const int ca = i0 + lc4 < P ? i0 + lc4 : 0;
  const int cb = j0 + lc4 < Q ? j0 + lc4 : 0;
  // Rows past the group's end read its last row and are replaced by zeros
  // (a select of values: a select of pointers would read zeros from memory).
  float4 ra0, ra1, rb0, rb1;
#define PRICHS_WGF_SEL(v, ok) \
  v = make_float4((ok) ? v.x : 0.f, (ok) ? v.y : 0.f, (ok) ? v.z : 0.f, (ok) ? v.w : 0.f)
#define PRICHS_WGF_LOAD(k0)                                                         \
  do {                                                                              \
    const int r0_ = (k0) + lrow, r1_ = (k0) + lrow + 8;                             \
    const size_t s0_ = (size_t)(row_lo + min(r0_, mg - 1));                         \
    const size_t s1_ = (size_t)(row_lo + min(r1_, mg - 1));                         \
    ra0 = *reinterpret_cast<const float4 *>(A + s0_ * lda + ca);                    \
    rb0 = *reinterpret_cast<const float4 *>(B + s0_ * ldb + cb);                    \
    ra1 = *reinterpret_cast<const float4 *>(A + s1_ * lda + ca);                    \
    rb1 = *reinterpret_cast<const float4 *>(B + s1_ * ldb + cb);                    \
    PRICHS_WGF_SEL(ra0, r0_ < mg);                                                  \
    PRICHS_WGF_SEL(rb0, r0_ < mg);                                                  \
    PRICHS_WGF_SEL(ra1, r1_ < mg);                                                  \
    PRICHS_WGF_SEL(rb1, r1_ < mg);                                                  \
  } while (0)
#define PRICHS_WGF_STORE(buf)                                             \
  do {                                                                    \
    float *as_ = ldsw + (buf) * 2 * kTile;                                \
    float *bs_ = as_ + kTile;                                             \
    *reinterpret_cast<float4 *>(as_ + lrow * kLd + lc4) = ra0;            \
    *reinterpret_cast<float4 *>(bs_ + lrow * kLd + lc4) = rb0;            \
    *reinterpret_cast<float4 *>(as_ + (lrow + 8) * kLd + lc4) = ra1;      \
    *reinterpret_cast<float4 *>(bs_ + (lrow + 8) * kLd + lc4) = rb1;      \
  } while (0)
  f32x4 acc[4][4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[j][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int KT = (mg + BK - 1) / BK;
  PRICHS_WGF_LOAD(0);
  PRICHS_WGF_STORE(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const bool more = kt + 1 < KT;
    if (more) PRICHS_WGF_LOAD((kt + 1) * BK);
    const float *as = ldsw + (kt & 1) * 2 * kTile;
    const float *bs = as + kTile;
#pragma unroll
    for (int ks = 0; ks < BK / 4; ++ks) {
      const int row = ks * 4 + (lane >> 4);
      float av[4], bv[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        av[b] = as[row * kLd + wp * 64 + b * 16 + (lane & 15)];
        bv[b] = bs[row * kLd + wq * 64 + b * 16 + (lane & 15)];
      }
#pragma unroll
      for (int jb = 0; jb < 4; ++jb)
#pragma unroll
        for (int ib = 0; ib < 4; ++ib)
          acc[jb][ib] = __builtin_amdgcn_mfma_f32_16x16x4f32(bv[jb], av[ib], acc[jb][ib], 0, 0, 0);
    }
    if (more) PRICHS_WGF_STORE((kt + 1) & 1);
    __syncthreads();
  }
#undef PRICHS_WGF_LOAD
#undef PRICHS_WGF_SEL
#undef PRICHS_WGF_STORE
  const long long base = (long long)slot_of(g, E) * slot_stride;
#pragma unroll
  for (int jb = 0; jb < 4; ++jb)
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) {
      const int i = i0 + wp * 64 + ib * 16 + (lane & 15);
      const int j = j0 + wq * 64 + jb * 16 + 4 * (lane >> 4);
      float *dst = wgrad_dst<GATEUP>(out0, out1, ldo, base, i, j, P, Q, f);
      if (dst) {
        float4 v = make_float4(acc[jb][ib][0], acc[jb][ib][1], acc[jb][ib][2], acc[jb][ib][3]);
        if (beta != 0) {
          const float4 o = *reinterpret_cast<const float4 *>(dst);
          v.x = o.x + v.x;
          v.y = o.y + v.y;
          v.z = o.z + v.z;
          v.w = o.w + v.w;
        }
        *reinterpret_cast<float4 *>(dst) = v;
      }
    }
}

// ------------------------------------------------------------- combine --
// Per token t (8 columns per thread): the router VJP of
// moe_router_unbiased_backward (backward.rs:269-287) over its k selections
// in selection order, ws = sum_j g_j s_j, d_logit_j = g_j (s_j - ws); then
//   d_x[t] = sum over the routed rows in ascending expert order of
//            (w_j if weighting == 2 else 1) * dX[row_j]
//          + dX[shared row of t]
//          + sum over the selections in ascending expert order of
//            d_logit_j * W_router[:, e_j]
// (the reference's scatter_add_grad, kernels.cu:971-991, applies w_j to dX,
// whose dY already carried w_j; weighting = 1 is the chain rule).  W_router
// comes transposed, wrt [E, d], so a selection's 8 columns are one vector
// load.  The thread of column 0 also writes d_logit_j at the row of each
// selection (dlr [T*k], in row-space order) for the router's weight gradient.
// dX is read here for the last time, so its loads are non-temporal (training
// step -1.5 us: they leave the caches to dW_gate/up's operands).
// KC: the top-k as a compile-time constant (k = 1, 2), or 0 for k at run time.
template <typename T, typename OT, int KC>
__global__ __launch_bounds__(256) void combine_kernel(
    const T *__restrict__ dX, const float *__restrict__ scal, const int32_t *__restrict__ topk_idx,
    const float *__restrict__ topk_w, const int32_t *__restrict__ token_row,
    const float *__restrict__ wrt, int T_, int d, int k_rt, int weighting,
    float *__restrict__ dlr, OT *__restrict__ d_x) {
#pragma clang fp contract(off)
  constexpr int kMax = KC > 0 ? KC : PRICHS_MAX_TOPK;
  const int k = KC > 0 ? KC : k_rt;
  const int per_tok = d / 8;
  const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (long long)T_ * per_tok) return;
  const int t = (int)(gid / per_tok);
  const int c = (int)(gid - (long long)t * per_tok) * 8;

  int ex[kMax], rows[kMax];
  float wt[kMax], dl[kMax];
  float ws = 0.f;
#pragma unroll
  for (int s = 0; s < kMax; ++s) {
    if (s < k) {
      ex[s] = topk_idx[(size_t)t * k + s];
      rows[s] = token_row[(size_t)t * k + s];
      wt[s] = topk_w[(size_t)t * k + s];
      dl[s] = scal[rows[s]];
      const float p = wt[s] * dl[s];
      ws = ws + p;
    } else {
      ex[s] = 0x7fffffff;
      rows[s] = 0;
      wt[s] = 0.f;
      dl[s] = 0.f;
    }
  }
#pragma unroll
  for (int s = 0; s < kMax; ++s) {
    const float diff = dl[s] - ws;
    dl[s] = s < k ? wt[s] * diff : 0.f;
  }
  // Ascending expert id (bubble passes over registers, as in the forward combine).
#pragma unroll
  for (int a = 0; a < kMax - 1; ++a)
#pragma unroll
    for (int b = 0; b < kMax - 1 - a; ++b)
      if (ex[b] > ex[b + 1]) {
        int te = ex[b]; ex[b] = ex[b + 1]; ex[b + 1] = te;
        int tr = rows[b]; rows[b] = rows[b + 1]; rows[b + 1] = tr;
        float tw = wt[b]; wt[b] = wt[b + 1]; wt[b + 1] = tw;
        float td = dl[b]; dl[b] = dl[b + 1]; dl[b + 1] = td;
      }
  if (c == 0) {
#pragma unroll
    for (int s = 0; s < kMax; ++s)
      if (s < k) dlr[rows[s]] = dl[s];
  }
  float acc[8], v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.f;
#pragma unroll
  for (int s = 0; s < kMax; ++s) {
    if (s < k) {
      V8<T>::load_nt(dX + (size_t)rows[s] * d + c, v);
      const float wx = weighting == 2 ? wt[s] : 1.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float p = wx * v[j];
        acc[j] = acc[j] + p;
      }
    }
  }
  V8<T>::load_nt(dX + ((size_t)T_ * k + t) * d + c, v);
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = acc[j] + v[j];
  float rs[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) rs[j] = 0.f;
#pragma unroll
  for (int s = 0; s < kMax; ++s) {
    if (s < k) {
      V8<float>::load(wrt + (size_t)ex[s] * d + c, v);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float p = dl[s] * v[j];
        rs[j] = rs[j] + p;
      }
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = acc[j] + rs[j];
  V8<OT>::store(d_x + (size_t)t * d + c, acc);
}

// ------------------------------------------------------- router weights --
// dW_router [d, E] += x^T d_logits (the reference's router sgemm, beta = 1,
// engine.rs:2705-2789).  d_logits[t][e] is zero unless t selected e, so
// column e is a weighted sum over expert e's rows of the row space:
// dW[:, e] += sum over rows r of group e of dlr[r] * xg[r] (xg = x gathered
// by row, written by the rows pass).  Pass 1: one workgroup per chunk of
// kRouterChunk rows of one group (chunks numbered group by group) writes
// part[chunk][c]; pass 2 adds each group's chunks in ascending order.
constexpr int kRouterChunk = 64;
constexpr int kRouterUnroll = 8;  // rows whose loads are in flight together

// Group and row range of chunk `ch` (-1 past the last chunk); offsets in LDS.
__device__ inline int router_chunk(const int *offsets, int E, int ch, int &r0, int &r1) {
  int first = 0;
  for (int e = 0; e < E; ++e) {
    const int lo = offsets[e], hi = offsets[e + 1];
    const int n = (hi - lo + kRouterChunk - 1) / kRouterChunk;
    if (ch < first + n) {
      r0 = lo + (ch - first) * kRouterChunk;
      r1 = min(r0 + kRouterChunk, hi);
      return e;
    }
    first += n;
  }
  return -1;
}

template <typename T>
__global__ __launch_bounds__(256) void router_wgrad_part_kernel(const T *__restrict__ xg,
                                                                const float *__restrict__ dlr,
                                                                const int32_t *__restrict__ offsets,
                                                                int E, int d,
                                                                float *__restrict__ part) {
#pragma clang fp contract(off)
  __shared__ int offs_s[PRICHS_MAX_EXPERTS + 1];
  if ((int)threadIdx.x <= E) offs_s[threadIdx.x] = offsets[threadIdx.x];
  __syncthreads();
  int r0 = 0, r1 = 0;
  if (router_chunk(offs_s, E, blockIdx.x, r0, r1) < 0) return;
  for (int c = threadIdx.x * 8; c < d; c += 256 * 8) {
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.f;
    for (int r = r0; r < r1; r += kRouterUnroll) {
      float xv[kRouterUnroll][8], w[kRouterUnroll];
#pragma unroll
      for (int u = 0; u < kRouterUnroll; ++u) {
        const int rr = min(r + u, r1 - 1);  // rows past r1 get weight 0 below
        V8<T>::load(xg + (size_t)rr * d + c, xv[u]);
        w[u] = r + u < r1 ? dlr[rr] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < kRouterUnroll; ++u)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float p = xv[u][j] * w[u];
          acc[j] = acc[j] + p;
        }
    }
    V8<float>::store(part + (size_t)blockIdx.x * d + c, acc);
  }
}

__global__ __launch_bounds__(256) void router_wgrad_reduce_kernel(const float *__restrict__ part,
                                                                  const int32_t *__restrict__ offsets,
                                                                  int E, int d, int beta,
                                                                  float *__restrict__ dw) {
#pragma clang fp contract(off)
  __shared__ int offs_s[PRICHS_MAX_EXPERTS + 1];
  if ((int)threadIdx.x <= E) offs_s[threadIdx.x] = offsets[threadIdx.x];
  __syncthreads();
  // Column-fastest (a wave's loads of one chunk row are contiguous), the
  // chunks of the column's group added in order, 16 loads in flight.
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= d * E) return;
  const int e = i / d, c = i - e * d;
  int first = 0;
  for (int g = 0; g < e; ++g)
    first += (offs_s[g + 1] - offs_s[g] + kRouterChunk - 1) / kRouterChunk;
  const int n = (offs_s[e + 1] - offs_s[e] + kRouterChunk - 1) / kRouterChunk;
  float s = 0.f;
  for (int ch = 0; ch < n; ch += 16) {
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u)
      v[u] = part[(size_t)(first + min(ch + u, n - 1)) * d + c];
#pragma unroll
    for (int u = 0; u < 16; ++u)
      if (ch + u < n) s = s + v[u];
  }
  const size_t o = (size_t)c * E + e;
  dw[o] = beta != 0 ? dw[o] + s : s;
}

unsigned blocks_for(long long n, int per = 256) { return (unsigned)((n + per - 1) / per); }

// Zeros of every gradient (beta = 0 with no rows): d_router [n_router], and
// per slot s < G the three [n_mat] matrices at slot_stride * s.
__global__ __launch_bounds__(256) void zero_grads_kernel(float *d_router, long long n_router,
                                                         float *d_gate, float *d_up, float *d_down,
                                                         long long slot_stride, int G,
                                                         long long n_mat) {
  const long long total = n_router + 3LL * G * n_mat;
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < total;
       i += (long long)gridDim.x * 256) {
    if (i < n_router) {
      d_router[i] = 0.f;
      continue;
    }
    const long long r = i - n_router;
    const long long which = r / (G * n_mat), q = r - which * G * n_mat;
    const long long slot = q / n_mat, e = q - slot * n_mat;
    float *m = which == 0 ? d_gate : which == 1 ? d_up : d_down;
    m[slot * slot_stride + e] = 0.f;
  }
}

// ---------------------------------------------------- legacy launchers --
// The reference's backward launchers with their exact f32 signatures
// (kernels.cu:498-514, 1026-1075; Rust extern block engine.rs:152-160,
// 244-271), so its per-expert backward links unchanged.  Same arithmetic as
// the reference kernels except: expf instead of __expf in the SwiGLU
// derivative, and the router dot as one wave per row summed in a fixed order
// (the reference's block reduction order is not part of its contract).

// kernels.cu:459-480.
__global__ __launch_bounds__(256) void legacy_swiglu_bwd_kernel(const float *__restrict__ dact,
                                                                const float *__restrict__ gate,
                                                                const float *__restrict__ up,
                                                                float *__restrict__ dgate,
                                                                float *__restrict__ dup, size_t n) {
#pragma clang fp contract(off)
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float g = gate[i], u = up[i], dy = dact[i];
  const float sig = 1.0f / (1.0f + expf(-g));
  const float silu = g * sig;
  const float dsilu = sig * (1.0f + g * (1.0f - sig));
  dup[i] = dy * silu;
  const float dyu = dy * u;
  dgate[i] = dyu * dsilu;
}

// kernels.cu:926-944: d_y_e[i][c] = w[i] * d_moe[idx[i]][c].
__global__ __launch_bounds__(256) void legacy_gather_weighted_kernel(
    const float *__restrict__ d_moe, const int *__restrict__ idx, const float *__restrict__ w,
    float *__restrict__ d_y_e, size_t n_tok, size_t hidden) {
#pragma clang fp contract(off)
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_tok * hidden) return;
  const size_t r = i / hidden, c = i - r * hidden;
  d_y_e[i] = w[r] * d_moe[(size_t)idx[r] * hidden + c];
}

// kernels.cu:946-969: scalars[i] = <exp_out[i], d_moe[idx[i]]>, one wave per row.
__global__ __launch_bounds__(256) void legacy_router_dot_kernel(
    const float *__restrict__ exp_out, const float *__restrict__ d_moe,
    const int *__restrict__ idx, float *__restrict__ scalars, size_t n_tok, size_t hidden) {
#pragma clang fp contract(off)
  const size_t r = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= n_tok) return;
  const float *a = exp_out + r * hidden;
  const float *b = d_moe + (size_t)idx[r] * hidden;
  float s = 0.f;
  for (size_t c = lane; c < hidden; c += 64) {
    const float p = a[c] * b[c];
    s = s + p;
  }
  s = wave_sum(s);
  if (lane == 0) scalars[r] = s;
}

// kernels.cu:971-991: d_normed2[idx[i]][c] += w[i] * (d_x_e[i][c] + d_x_e_tmp[i][c]),
// with the reference's atomic add (an expert's token list has distinct
// indices, so its use is order-free).
__global__ __launch_bounds__(256) void legacy_scatter_add_grad_kernel(
    const float *__restrict__ dxe, const float *__restrict__ dxe_tmp, const int *__restrict__ idx,
    const float *__restrict__ w, float *__restrict__ d_normed2, size_t n_tok, size_t hidden) {
#pragma clang fp contract(off)
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_tok * hidden) return;
  const size_t r = i / hidden, c = i - r * hidden;
  const float sum = dxe[i] + dxe_tmp[i];
  const float val = w[r] * sum;
  atomicAdd(d_normed2 + (size_t)idx[r] * hidden + c, val);
}

}  // namespace

// ---------------------------------------------------------------- launchers --
int bwd_rows(const void *x, const void *d_out, const void *y, const int32_t *token_row,
             const float *row_weight, size_t T, size_t k, bool shared, size_t d, int dtype,
             void *dy, void *xg, float *scal, hipStream_t s) {
  if (T == 0) return PRICHS_OK;
  const unsigned grid = (unsigned)cdiv(T, 4);  // one wave per token
#define PRICHS_ROWS_K(TT, KC)                                                                    \
  hipLaunchKernelGGL((rows_kernel<TT, KC>), dim3(grid), dim3(256), 0, s,                        \
                     static_cast<const TT *>(x), static_cast<const TT *>(d_out),                \
                     static_cast<const TT *>(y), token_row, row_weight, (int)T, (int)k, (int)d, \
                     shared ? 1 : 0, static_cast<TT *>(dy), static_cast<TT *>(xg), scal)
#define PRICHS_ROWS(TT)          \
  do {                           \
    if (k == 2)                  \
      PRICHS_ROWS_K(TT, 2);      \
    else if (k == 1)             \
      PRICHS_ROWS_K(TT, 1);      \
    else                         \
      PRICHS_ROWS_K(TT, 0);      \
  } while (0)
  if (dtype == PRICHS_DTYPE_BF16)
    PRICHS_ROWS(bf16_t);
  else
    PRICHS_ROWS(float);
#undef PRICHS_ROWS
#undef PRICHS_ROWS_K
  PRICHS_LAUNCH_CHECK("moe backward: rows");
  return PRICHS_OK;
}

int bwd_swiglu(void *gu, const void *da, size_t rows, size_t f, size_t np, int dtype,
               hipStream_t s) {
  if (rows == 0) return PRICHS_OK;
  const long long n = (long long)rows * (long long)(np / (2 * kIl) * (kIl / 8));
  if (dtype == PRICHS_DTYPE_BF16)
    hipLaunchKernelGGL(swiglu_bwd_kernel<bf16_t>, dim3(blocks_for(n)), dim3(256), 0, s,
                       static_cast<bf16_t *>(gu), static_cast<const bf16_t *>(da), (int)rows,
                       (int)f, (int)np);
  else
    hipLaunchKernelGGL(swiglu_bwd_kernel<float>, dim3(blocks_for(n)), dim3(256), 0, s,
                       static_cast<float *>(gu), static_cast<const float *>(da), (int)rows,
                       (int)f, (int)np);
  PRICHS_LAUNCH_CHECK("moe backward: swiglu");
  return PRICHS_OK;
}

// A split group has m > kSplitRows rows and at most ceil(m / kSplitRows) <=
// 2 floor(m / kSplitRows) chunks, so all split groups together hold at most
// 2 floor(rows / kSplitRows) chunk partials.
size_t bwd_wgrad_part_elems(size_t max_rows, size_t P, size_t Q) {
  return 2 * (max_rows / wgb::kSplitRows) * P * Q;
}

int bwd_wgrad(bool gateup, const void *A, size_t lda, const void *B, size_t ldb, size_t total_rows,
              const int32_t *offsets, size_t G, size_t E, size_t P, size_t Q, float *out0,
              float *out1, size_t ldo, size_t slot_stride, size_t f, int dtype, float *part,
              int beta, hipStream_t s, const WgradAlt &alt) {
  if (total_rows == 0) return PRICHS_OK;
  const int cus = device_cu_count();
  const unsigned rgrid = (unsigned)std::max(1, 4 * cus);
  if (dtype == PRICHS_DTYPE_BF16) {
    const int tiles_q = (int)cdiv(Q, wgb::BQ);
    const int tiles = (int)cdiv(P, wgb::BP) * tiles_q;
    // Every group's chunks: at most G + total_rows / kSplitRows per tile.
    const size_t items = (G + total_rows / wgb::kSplitRows) * (size_t)tiles;
    const size_t ab = total_rows * lda * 2, bb = total_rows * ldb * 2;
    const size_t ab2 = alt.A ? alt.rows * lda * 2 : 0, bb2 = alt.B ? alt.rows * ldb * 2 : 0;
    if (ab >= wgb::kOutOfRange || bb >= wgb::kOutOfRange || ab2 >= wgb::kOutOfRange ||
        bb2 >= wgb::kOutOfRange || P * Q * 4 >= wgb::kOutOfRange)
      return fail(PRICHS_ERR_UNSUPPORTED,
                  "moe backward: operands of %zu and %zu bytes or a %zu x %zu gradient exceed 2 GiB",
                  ab, bb, P, Q);
    if (items + (size_t)cus > (size_t)INT32_MAX)
      return fail(PRICHS_ERR_UNSUPPORTED, "moe backward: too many tiles");
    auto kern = gateup ? wgrad_bf16_kernel<true, false> : wgrad_bf16_kernel<false, true>;
    static bool attr_set[2] = {false, false};
    if (!attr_set[gateup]) {
      PRICHS_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize,
                                         (int)wgb::kLdsBytes),
                     "moe backward: set LDS size");
      attr_set[gateup] = true;
    }
    // The item bound plus half a round: a last round of at most cus / 2
    // items may run as twice as many half-height items.  (Workgroups past
    // the items exit at once, but each still waits for a free CU.)
    const bool halves = !gateup;  // dW_down (see wgrad_bf16_kernel)
    const size_t grid = items + (halves ? (size_t)(cus / 2) : 0);
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(wgb::kThreads), wgb::kLdsBytes, s,
                       static_cast<const bf16_t *>(A), (int)lda, (uint32_t)ab,
                       static_cast<const bf16_t *>(B), (int)ldb, (uint32_t)bb, offsets, (int)G,
                       (int)E, (int)P, (int)Q, tiles_q, tiles, out0, out1, (int)ldo,
                       (long long)slot_stride, (int)f, part, beta, cus,
                       static_cast<const bf16_t *>(alt.A), (uint32_t)ab2,
                       static_cast<const bf16_t *>(alt.B), (uint32_t)bb2,
                       alt.A || alt.B ? (int)alt.g : -1, (int)alt.row0);
    PRICHS_LAUNCH_CHECK("moe backward: weight gradient");
    // Some group may have been split, or (beta = 0) may have no rows.
    if (total_rows > (size_t)wgb::kSplitRows || beta == 0) {
      auto rk = gateup ? wgrad_reduce_kernel<true> : wgrad_reduce_kernel<false>;
      hipLaunchKernelGGL(rk, dim3(rgrid), dim3(256), 0, s, part, offsets, (int)G, (int)E, (int)P,
                         (int)Q, out0, out1, (int)ldo, (long long)slot_stride, (int)f, beta, 1);
      PRICHS_LAUNCH_CHECK("moe backward: weight gradient partials");
    }
    return PRICHS_OK;
  }
  if (alt.A || alt.B)
    return fail(PRICHS_ERR_UNSUPPORTED, "moe backward: alternate row buffers need bf16");
  const int tiles_q = (int)cdiv(Q, wg::BQ);
  const int tiles = (int)cdiv(P, wg::BP) * tiles_q;
  const unsigned grid = (unsigned)(8 * cdiv((size_t)tiles, 8) * G);
  auto kern = gateup ? wgrad_f32_kernel<true> : wgrad_f32_kernel<false>;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(wg::kThreads), wgf::kLdsBytes, s,
                     static_cast<const float *>(A), (int)lda, static_cast<const float *>(B),
                     (int)ldb, offsets, (int)G, (int)E, (int)P, (int)Q, tiles_q, tiles, out0,
                     out1, (int)ldo, (long long)slot_stride, (int)f, beta);
  PRICHS_LAUNCH_CHECK("moe backward: weight gradient");
  if (beta == 0) {  // zeros for groups without rows
    auto rk = gateup ? wgrad_reduce_kernel<true> : wgrad_reduce_kernel<false>;
    hipLaunchKernelGGL(rk, dim3(rgrid), dim3(256), 0, s, nullptr, offsets, (int)G, (int)E, (int)P,
                       (int)Q, out0, out1, (int)ldo, (long long)slot_stride, (int)f, 0, 0);
    PRICHS_LAUNCH_CHECK("moe backward: weight gradient zeros");
  }
  return PRICHS_OK;
}

int bwd_combine(const void *dX, const float *scal, const int32_t *topk_idx, const float *topk_w,
                const int32_t *token_row, const float *wrt, size_t T, size_t d, size_t k,
                int weighting, int dtype, float *dlr, void *d_x, int dx_dtype, hipStream_t s) {
  if (T == 0) return PRICHS_OK;
  const unsigned grid = blocks_for((long long)T * (long long)(d / 8));
#define PRICHS_BWD_COMBINE_K(TT, OT, KC)                                                        \
  hipLaunchKernelGGL((combine_kernel<TT, OT, KC>), dim3(grid), dim3(256), 0, s,                \
                     static_cast<const TT *>(dX), scal, topk_idx, topk_w, token_row, wrt,      \
                     (int)T, (int)d, (int)k, weighting, dlr, static_cast<OT *>(d_x))
#define PRICHS_BWD_COMBINE(TT, OT)         \
  do {                                     \
    if (k == 2)                            \
      PRICHS_BWD_COMBINE_K(TT, OT, 2);     \
    else if (k == 1)                       \
      PRICHS_BWD_COMBINE_K(TT, OT, 1);     \
    else                                   \
      PRICHS_BWD_COMBINE_K(TT, OT, 0);     \
  } while (0)
  if (dtype == PRICHS_DTYPE_BF16) {
    if (dx_dtype == PRICHS_DTYPE_BF16)
      PRICHS_BWD_COMBINE(bf16_t, bf16_t);
    else
      PRICHS_BWD_COMBINE(bf16_t, float);
  } else {
    if (dx_dtype == PRICHS_DTYPE_BF16)
      PRICHS_BWD_COMBINE(float, bf16_t);
    else
      PRICHS_BWD_COMBINE(float, float);
  }
#undef PRICHS_BWD_COMBINE
#undef PRICHS_BWD_COMBINE_K
  PRICHS_LAUNCH_CHECK("moe backward: combine");
  return PRICHS_OK;
}

int bwd_zero_grads(float *d_router, size_t n_router, float *d_gate, float *d_up, float *d_down,
                   size_t slot_stride, size_t G, size_t n_mat, hipStream_t s) {
  const int cus = device_cu_count();
  hipLaunchKernelGGL(zero_grads_kernel, dim3((unsigned)std::max(1, 4 * cus)), dim3(256), 0, s,
                     d_router, (long long)n_router, d_gate, d_up, d_down, (long long)slot_stride,
                     (int)G, (long long)n_mat);
  PRICHS_LAUNCH_CHECK("moe backward: zero gradients");
  return PRICHS_OK;
}

size_t bwd_router_part_elems(size_t max_tokens, size_t k, size_t d, size_t E) {
  return (cdiv(max_tokens * k, kRouterChunk) + E) * d;
}

int bwd_router_wgrad(const void *xg, const float *dlr, const int32_t *offsets, size_t T, size_t k,
                     size_t d, size_t E, int dtype, float *part, float *dw, int beta,
                     hipStream_t s) {
  if (T == 0) return PRICHS_OK;
  // Every group's chunks fit in cdiv(T*k, chunk) + E workgroups; the rest exit.
  const unsigned grid = (unsigned)(cdiv(T * k, kRouterChunk) + E);
  if (dtype == PRICHS_DTYPE_BF16)
    hipLaunchKernelGGL(router_wgrad_part_kernel<bf16_t>, dim3(grid), dim3(256), 0, s,
                       static_cast<const bf16_t *>(xg), dlr, offsets, (int)E, (int)d, part);
  else
    hipLaunchKernelGGL(router_wgrad_part_kernel<float>, dim3(grid), dim3(256), 0, s,
                       static_cast<const float *>(xg), dlr, offsets, (int)E, (int)d, part);
  PRICHS_LAUNCH_CHECK("moe backward: router weight gradient");
  hipLaunchKernelGGL(router_wgrad_reduce_kernel, dim3(blocks_for((long long)(d * E))), dim3(256),
                     0, s, part, offsets, (int)E, (int)d, beta, dw);
  PRICHS_LAUNCH_CHECK("moe backward: router weight gradient reduce");
  return PRICHS_OK;
}

}  // namespace prichs

using namespace prichs;

extern "C" void launch_swiglu_backward(const float *dev_dact, const float *dev_gate,
                                       const float *dev_up, float *dev_dgate, float *dev_dup,
                                       size_t total_elements, void *stream) {
  if (total_elements == 0) return;
  if (!dev_dact || !dev_gate || !dev_up || !dev_dgate || !dev_dup) {
    set_error("launch_swiglu_backward: null pointer argument");
    return;
  }
  hipLaunchKernelGGL(legacy_swiglu_bwd_kernel, dim3(blocks_for((long long)total_elements)),
                     dim3(256), 0, as_stream(stream), dev_dact, dev_gate, dev_up, dev_dgate,
                     dev_dup, total_elements);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) set_error("launch_swiglu_backward: %s", hipGetErrorString(e));
}

extern "C" void launch_moe_backward_gather_weighted(const float *dev_d_moe,
                                                    const int *dev_token_indices,
                                                    const float *dev_weights, float *dev_d_y_e,
                                                    size_t n_tokens, size_t hidden_dim,
                                                    void *stream) {
  const size_t n = n_tokens * hidden_dim;
  if (n == 0) return;
  if (!dev_d_moe || !dev_token_indices || !dev_weights || !dev_d_y_e) {
    set_error("launch_moe_backward_gather_weighted: null pointer argument");
    return;
  }
  hipLaunchKernelGGL(legacy_gather_weighted_kernel, dim3(blocks_for((long long)n)), dim3(256), 0,
                     as_stream(stream), dev_d_moe, dev_token_indices, dev_weights, dev_d_y_e,
                     n_tokens, hidden_dim);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) set_error("launch_moe_backward_gather_weighted: %s", hipGetErrorString(e));
}

extern "C" void launch_moe_router_dot(const float *dev_exp_out, const float *dev_d_moe,
                                      const int *dev_token_indices, float *dev_scalars_out,
                                      size_t n_tokens, size_t hidden_dim, void *stream) {
  if (n_tokens == 0) return;
  if (!dev_exp_out || !dev_d_moe || !dev_token_indices || !dev_scalars_out) {
    set_error("launch_moe_router_dot: null pointer argument");
    return;
  }
  hipLaunchKernelGGL(legacy_router_dot_kernel, dim3((unsigned)cdiv(n_tokens, 4)), dim3(256), 0,
                     as_stream(stream), dev_exp_out, dev_d_moe, dev_token_indices,
                     dev_scalars_out, n_tokens, hidden_dim);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) set_error("launch_moe_router_dot: %s", hipGetErrorString(e));
}

extern "C" void launch_moe_scatter_add_grad(const float *dev_d_x_e, const float *dev_d_x_e_tmp,
                                            const int *dev_token_indices,
                                            const float *dev_weights, float *dev_d_normed2,
                                            size_t n_tokens, size_t hidden_dim, void *stream) {
  const size_t n = n_tokens * hidden_dim;
  if (n == 0) return;
  if (!dev_d_x_e || !dev_d_x_e_tmp || !dev_token_indices || !dev_weights || !dev_d_normed2) {
    set_error("launch_moe_scatter_add_grad: null pointer argument");
    return;
  }
  hipLaunchKernelGGL(legacy_scatter_add_grad_kernel, dim3(blocks_for((long long)n)), dim3(256), 0,
                     as_stream(stream), dev_d_x_e, dev_d_x_e_tmp, dev_token_indices, dev_weights,
                     dev_d_normed2, n_tokens, hidden_dim);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) set_error("launch_moe_scatter_add_grad: %s", hipGetErrorString(e));
}
