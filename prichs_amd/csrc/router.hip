// router.hip -- router logits + top-k gating, and the token permutation.
//
// Router: restates crates/prichs-model/src/moe.rs:113-142 and
// crates/prichs-core/src/ops.rs:219-248 on device.  One lane owns one
// (token, expert) logit and accumulates it in the reference CPU GEMM's order
// (k ascending, product rounded then sum rounded, crates/prichs-core/src/
// ops.rs:49-56), so logits -- and therefore every routing decision -- are
// bit-exact with the reference CPU path.  The lanes of one token form a
// power-of-two group inside a wave64; top-k is k rounds of a butterfly
// arg-max over that group.
//
// Permutation: a stable counting sort by expert id.  The router emits a
// per-block expert histogram; each permutation block sums the histograms of
// the blocks before it (exclusive scan) and places its own tokens in token
// order, which yields the reference's (expert ascending, token ascending)
// binning order (moe.rs:121, 137-141, 149) without atomics on the output.
#include "common.hpp"
#include "router_quad.hpp"

namespace prichs {

namespace {

using namespace rq;  // kRouterThreads, topk_epilogue, place_entries, FusedPerm, the quad body

// Quad-broadcast router for E <= 8 (1) or always the staged router (0).
#ifndef PRICHS_ROUTER_QUAD
#define PRICHS_ROUTER_QUAD 1
#endif
constexpr int kRouterLdsBytes = 60 * 1024;  // simple kernel: W chunk [E][kc + 4] f32

int lanes_per_token_log2(int E) {
  int l = 0;
  while ((1 << l) < E) ++l;
  return l;
}

// Width of the router-weight chunk of the simple kernel.
int router_chunk(int d, int E) {
  int kc = (kRouterLdsBytes / 4) / E - 4;
  kc = kc / 8 * 8;
  int dpad = (d + 7) / 8 * 8;
  return kc < dpad ? kc : dpad;
}

// ---------------------------------------------------------------------------
// Staged router: the block's x rows and router weights go through
// double-buffered LDS in K chunks of KC (coalesced 16-byte loads by all 256
// threads, one chunk in flight while the previous one is summed), and each
// lane then sums its (token, expert) dot product over k in ascending order,
// product rounded then sum rounded -- the reference CPU GEMM's order
// (crates/prichs-core/src/ops.rs:49-56).  LPT lanes per token (LPT >= E).
// Requires d % 8 == 0 and 16-byte aligned x and W.
// ---------------------------------------------------------------------------
template <typename XT, int LPT, int KC> struct StagedRouter {
  static constexpr int kTpb = kRouterThreads / LPT;  // tokens per block
  static constexpr int kVe = 16 / (int)sizeof(XT);   // x elements per 16-byte load
  static constexpr int kXStride = KC + 4;            // f32 x row in LDS (16-byte pad)
  static constexpr int kWStride = KC + 4;            // W^T row in LDS
  static constexpr int kXTot = kTpb * KC / kVe;      // x vectors per chunk
  static constexpr int kXVec = (kXTot + kRouterThreads - 1) / kRouterThreads;
  static constexpr int kWVec = (KC * LPT / 4 + kRouterThreads - 1) / kRouterThreads;
  static constexpr size_t kXBytes = (size_t)kTpb * kXStride * sizeof(float);
  static constexpr size_t kWBytes = (size_t)LPT * kWStride * sizeof(float);
  static constexpr size_t kLds = 2 * (kXBytes + kWBytes);
  static_assert(KC % 8 == 0 && (KC / kVe) > 0, "chunks of whole 16-byte vectors");
};


// Global -> registers: x rows tok0.. of chunk k0 and the chunk's W rows [n][E]
// as float4s.  No load is predicated (a predicated load makes the compiler
// drain every load in flight at the join): rows past T read row T-1, vectors
// past the chunk re-read the chunk's last vector, and the values so fetched
// are never summed.
template <typename XT, int LPT, int KC>
__device__ inline void router_fetch(const XT *__restrict__ x, const float *__restrict__ w,
                                    int tid, int tok0, int T, int d, int E, int k0, int n,
                                    u32x4 (&rx)[StagedRouter<XT, LPT, KC>::kXVec],
                                    f32x4 (&rw)[StagedRouter<XT, LPT, KC>::kWVec]) {
  using Cf = StagedRouter<XT, LPT, KC>;
  constexpr int vpr = KC / Cf::kVe;
#pragma unroll
  for (int i = 0; i < Cf::kXVec; ++i) {
    const int v = min(tid + kRouterThreads * i, Cf::kXTot - 1);
    const int r = v / vpr, cv = v % vpr;
    const int row = min(tok0 + r, T - 1);
    const int col = min(cv * Cf::kVe, n - Cf::kVe);
    rx[i] = *reinterpret_cast<const u32x4 *>(x + (size_t)row * d + k0 + col);
  }
  const int nw = n * E / 4;  // n is a multiple of 8, so whole float4s
#pragma unroll
  for (int i = 0; i < Cf::kWVec; ++i) {
    const int v = min(tid + kRouterThreads * i, nw - 1);
    rw[i] = *reinterpret_cast<const f32x4 *>(w + (size_t)k0 * E + 4 * v);
  }
}

// Registers -> LDS: x as f32 rows (bf16 widened once here rather than by each
// of the token's lanes), W transposed to [e][k].
template <typename XT, int LPT, int KC>
__device__ inline void router_stash(float *__restrict__ xs, float *__restrict__ ws, int tid, int E,
                                    int n, const u32x4 (&rx)[StagedRouter<XT, LPT, KC>::kXVec],
                                    const f32x4 (&rw)[StagedRouter<XT, LPT, KC>::kWVec]) {
  using Cf = StagedRouter<XT, LPT, KC>;
  constexpr int vpr = KC / Cf::kVe;
#pragma unroll
  for (int i = 0; i < Cf::kXVec; ++i) {
    const int v = tid + kRouterThreads * i;
    const int r = v / vpr, cv = v % vpr;
    if (v < Cf::kXTot && cv * Cf::kVe < n) {
      float *dst = xs + r * Cf::kXStride + cv * Cf::kVe;
      if constexpr (sizeof(XT) == 2) {
        f32x4 lo, hi;
        lo.x = __uint_as_float(rx[i].x << 16);
        lo.y = __uint_as_float(rx[i].x & 0xffff0000u);
        lo.z = __uint_as_float(rx[i].y << 16);
        lo.w = __uint_as_float(rx[i].y & 0xffff0000u);
        hi.x = __uint_as_float(rx[i].z << 16);
        hi.y = __uint_as_float(rx[i].z & 0xffff0000u);
        hi.z = __uint_as_float(rx[i].w << 16);
        hi.w = __uint_as_float(rx[i].w & 0xffff0000u);
        *reinterpret_cast<f32x4 *>(dst) = lo;
        *reinterpret_cast<f32x4 *>(dst + 4) = hi;
      } else {
        f32x4 v4;
        v4.x = __uint_as_float(rx[i].x);
        v4.y = __uint_as_float(rx[i].y);
        v4.z = __uint_as_float(rx[i].z);
        v4.w = __uint_as_float(rx[i].w);
        *reinterpret_cast<f32x4 *>(dst) = v4;
      }
    }
  }
  const int nw = n * E / 4;
#pragma unroll
  for (int i = 0; i < Cf::kWVec; ++i) {
    const int v = tid + kRouterThreads * i;
    if (v < nw) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int f = 4 * v + j;  // flat index in [n][E]
        const int kk = f / E, ee = f - kk * E;
        ws[ee * Cf::kWStride + kk] = rw[i][j];
      }
    }
  }
}

// acc + x[0]*w[0] + ... + x[3]*w[3], each product and each sum rounded in turn.
__device__ inline float router_dot4(float acc, const float *xr, const float *wr) {
#pragma clang fp contract(off)
  const f32x4 xv = *reinterpret_cast<const f32x4 *>(xr);
  const f32x4 wv = *reinterpret_cast<const f32x4 *>(wr);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float p = xv[q] * wv[q];
    acc = acc + p;
  }
  return acc;
}

// Sum over one whole chunk, fully unrolled so the chunk's LDS reads are issued
// ahead of the dependent adds (at one wave per SIMD nothing else covers their
// latency).  With PRICHS_ROUTER_PIPE=1 (default; ~5% faster at config 2) a
// sched_group_barrier sequence also pins a read-ahead interleave (masks: 0x100
// LDS read, 0x2 VALU).  Either way the arithmetic order is the reference's:
// each product rounded, then each sum.
#ifndef PRICHS_ROUTER_PIPE
#define PRICHS_ROUTER_PIPE 1
#endif
template <int KC>
__device__ inline float router_dot_chunk(float acc, const float *xr, const float *wr) {
#pragma clang fp contract(off)
  constexpr int kG = KC / 4;
#if PRICHS_ROUTER_PIPE
  constexpr int kAhead = kG < 6 ? kG : 6;
  __builtin_amdgcn_sched_barrier(0);
#endif
#pragma unroll
  for (int g = 0; g < kG; ++g) {
    const f32x4 xv = *reinterpret_cast<const f32x4 *>(xr + 4 * g);
    const f32x4 wv = *reinterpret_cast<const f32x4 *>(wr + 4 * g);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float p = xv[q] * wv[q];
      acc = acc + p;
    }
  }
#if PRICHS_ROUTER_PIPE
  __builtin_amdgcn_sched_group_barrier(0x100, 2 * kAhead, 0);
#pragma unroll
  for (int g = 0; g < kG; ++g) {
    __builtin_amdgcn_sched_group_barrier(0x2, 8, 0);
    if (g + kAhead < kG) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
#endif
  return acc;
}

// waves_per_eu: the dynamic LDS holds a CU to a few blocks, so the compiler may
// spend registers on the read-ahead.
template <typename XT, int LPT, int KC>
__global__ __launch_bounds__(kRouterThreads) __attribute__((amdgpu_waves_per_eu(1, 3))) void
router_topk_staged_kernel(
    const XT *__restrict__ x, const float *__restrict__ w, const float *__restrict__ bias,
    const float *__restrict__ concept, int n_concept, int T, int d, int E, int k,
    float *__restrict__ logits, int32_t *__restrict__ topk_idx, float *__restrict__ topk_w,
    int32_t *__restrict__ block_counts) {
#pragma clang fp contract(off)
  using Cf = StagedRouter<XT, LPT, KC>;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  __shared__ int cnt_s[PRICHS_MAX_EXPERTS];
  float *const xs0 = reinterpret_cast<float *>(smem);
  float *const ws0 = reinterpret_cast<float *>(smem + Cf::kXBytes);
  constexpr size_t kBuf = (Cf::kXBytes + Cf::kWBytes) / sizeof(float);

  const int tid = threadIdx.x;
  const int e = tid & (LPT - 1);
  const int tl = tid / LPT;
  const int tok0 = blockIdx.x * Cf::kTpb;
  const int t = tok0 + tl;
  const bool valid = (t < T) && (e < E);
  if (tid < E) cnt_s[tid] = 0;
  const int n_chunks = (d + KC - 1) / KC;

  // Register ring of kRing chunks in flight: with one wave per SIMD at the
  // headline shape, nothing else hides HBM latency.
  constexpr int kRing = 4;
  u32x4 rx[kRing][Cf::kXVec];
  f32x4 rw[kRing][Cf::kWVec];
  auto chunk_len = [&](int c) { return min(KC, d - c * KC); };
  // Chunks past the end are fetched as the last chunk (unpredicated loads).
  auto fetch = [&](int c, u32x4(&rxs)[Cf::kXVec], f32x4(&rws)[Cf::kWVec]) {
    const int cc = min(c, n_chunks - 1);
    router_fetch<XT, LPT, KC>(x, w, tid, tok0, T, d, E, cc * KC, chunk_len(cc), rxs, rws);
  };
#pragma unroll
  for (int j = 0; j < kRing; ++j) fetch(j, rx[j], rw[j]);
  router_stash<XT, LPT, KC>(xs0, ws0, tid, E, chunk_len(0), rx[0], rw[0]);
  fetch(kRing, rx[0], rw[0]);
  __syncthreads();

  // Iteration c sums chunk c from LDS, stashes chunk c + 1 from its register
  // slot into the other LDS buffer and refills that slot with chunk
  // c + 1 + kRing.  The refill is issued on every path (only LDS work is
  // guarded) so the compiler's wait before each stash counts exactly the
  // loads issued after the slot's own.
  float acc = 0.0f;
  for (int c0 = 0; c0 < n_chunks; c0 += kRing) {
#pragma unroll
    for (int j = 0; j < kRing; ++j) {
      const int c = c0 + j;
      const int jn = (j + 1) % kRing;  // slot holding chunk c + 1
      if (valid && c < n_chunks) {
        const int n = chunk_len(c);
        const size_t off = (c & 1) * kBuf;
        const float *xr = xs0 + off + tl * Cf::kXStride;
        const float *wr = ws0 + off + e * Cf::kWStride;
        if (n == KC) {
          acc = router_dot_chunk<KC>(acc, xr, wr);
        } else {
          for (int kk = 0; kk < n; kk += 4) acc = router_dot4(acc, xr + kk, wr + kk);
        }
      }
      if (c + 1 < n_chunks) {
        const size_t noff = ((c + 1) & 1) * kBuf;
        router_stash<XT, LPT, KC>(xs0 + noff, ws0 + noff, tid, E, chunk_len(c + 1), rx[jn],
                                  rw[jn]);
      }
      fetch(c + 1 + kRing, rx[jn], rw[jn]);
      __syncthreads();
    }
  }

  // adj = (raw + bias[e]) (+ concept[e]), moe.rs:126-133.
  float adj = 0.0f;
  if (valid) {
    adj = acc + bias[e];
    if (concept != nullptr && e < n_concept) adj = adj + concept[e];
  }
  topk_epilogue(acc, adj, valid, e, t, T, E, k, LPT, logits, topk_idx, topk_w, cnt_s);
  __syncthreads();
  if (tid < E) block_counts[(size_t)blockIdx.x * E + tid] = cnt_s[tid];
}

// The quad-broadcast router (router_quad.hpp): one workgroup per 32 tokens.
template <typename XT>
__global__ __launch_bounds__(kRouterThreads) void router_topk_quad_kernel(
    const XT *__restrict__ x, const float *__restrict__ w, const float *__restrict__ bias,
    const float *__restrict__ concept, int n_concept, int T, int d, int E, int k,
    float *__restrict__ logits, int32_t *__restrict__ topk_idx, float *__restrict__ topk_w,
    int32_t *__restrict__ block_counts, FusedPerm perm, const float *__restrict__ w_lds) {
  extern __shared__ __attribute__((aligned(16))) float wt_s[];  // W^T [8][d + 4]
  router_quad_body<XT>(x, w, bias, concept, n_concept, T, d, E, k, logits, topk_idx, topk_w,
                       block_counts, perm, w_lds, (int)blockIdx.x, wt_s);
}

template <typename XT>
int launch_quad_t(const XT *x, const float *w, const float *bias, const float *concept, int nc,
                  int T, int d, int E, int k, float *logits, int32_t *idx, float *wt, int32_t *bc,
                  int nb, hipStream_t s, FusedPerm perm = FusedPerm{nullptr, nullptr, nullptr, nullptr},
                  const float *w_lds = nullptr) {
  const size_t lds = (size_t)8 * (d + 4) * sizeof(float);
  static int attr_bytes = 0;
  if ((int)lds > attr_bytes) {
    PRICHS_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void *>(&router_topk_quad_kernel<XT>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                   "router: set LDS size");
    attr_bytes = (int)lds;
  }
  hipLaunchKernelGGL((router_topk_quad_kernel<XT>), dim3(nb), dim3(kRouterThreads), lds, s, x, w,
                     bias, concept, nc, T, d, E, k, logits, idx, wt, bc, perm, w_lds);
  return PRICHS_OK;
}

// ---------------------------------------------------------------------------
// Simple router (any d): W chunks in LDS, x read straight from global.
// ---------------------------------------------------------------------------
template <typename XT>
__global__ __launch_bounds__(kRouterThreads) void router_topk_kernel(
    const XT *__restrict__ x, const float *__restrict__ w, const float *__restrict__ bias,
    const float *__restrict__ concept, int n_concept, int T, int d, int E, int k, int lpt_log2,
    int kc, float *__restrict__ logits, int32_t *__restrict__ topk_idx,
    float *__restrict__ topk_w, int32_t *__restrict__ block_counts) {
#pragma clang fp contract(off)
  extern __shared__ float w_s[];  // [E][kc + 4]
  __shared__ int cnt_s[PRICHS_MAX_EXPERTS];

  const int lpt = 1 << lpt_log2;
  const int tpb = kRouterThreads >> lpt_log2;
  const int tid = threadIdx.x;
  const int e = tid & (lpt - 1);
  const int t = blockIdx.x * tpb + (tid >> lpt_log2);
  const bool valid = (t < T) && (e < E);
  const int kcp = kc + 4;
  if (tid < E) cnt_s[tid] = 0;

  float acc = 0.0f;
  for (int k0 = 0; k0 < d; k0 += kc) {
    const int n = min(kc, d - k0);
    __syncthreads();
    for (int i = tid; i < n * E; i += kRouterThreads) {
      const int kk = i / E;
      const int ee = i - kk * E;
      w_s[ee * kcp + kk] = w[(size_t)(k0 + kk) * E + ee];
    }
    __syncthreads();
    if (valid) {
      const XT *xr = x + (size_t)t * d + k0;
      const float *wr = w_s + e * kcp;
      for (int kk = 0; kk < n; ++kk) {
        const float p = Elem<XT>::load(xr + kk) * wr[kk];
        acc = acc + p;
      }
    }
  }

  float adj = 0.0f;
  if (valid) {
    adj = acc + bias[e];
    if (concept != nullptr && e < n_concept) adj = adj + concept[e];
  }
  topk_epilogue(acc, adj, valid, e, t, T, E, k, lpt, logits, topk_idx, topk_w, cnt_s);
  __syncthreads();
  if (tid < E) block_counts[(size_t)blockIdx.x * E + tid] = cnt_s[tid];
}

__global__ void fill_i32_kernel(int32_t *p, int n, int v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

__global__ __launch_bounds__(256) void permute_kernel(
    const int32_t *__restrict__ topk_idx, const float *__restrict__ topk_w,
    const int32_t *__restrict__ block_counts, int T, int E, int k, int tpb,
    int nb, int32_t *__restrict__ offsets, int32_t *__restrict__ row_token,
    float *__restrict__ row_weight, int32_t *__restrict__ token_row) {
  __shared__ int tot_s[PRICHS_MAX_EXPERTS];
  __shared__ int pre_s[PRICHS_MAX_EXPERTS];
  __shared__ int base_s[PRICHS_MAX_EXPERTS];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  // This block's first 64 (token, slot) entries and its shared rows do not
  // depend on the histograms: their loads and stores go out first, so their
  // latency overlaps the histogram reads instead of following them.
  const int t0 = b * tpb, t1 = min(T, (b + 1) * tpb);
  const size_t s0 = (size_t)t0 * k, s1 = (size_t)t1 * k;
  const bool live0 = tid < 64 && s0 + tid < s1;
  const int e0 = live0 ? topk_idx[s0 + tid] : -1;
  const float w0 = live0 ? topk_w[s0 + tid] : 0.0f;
  for (int t = t0 + tid; t < t1; t += blockDim.x) row_token[(size_t)T * k + t] = t;
  if (tid < E) {
    tot_s[tid] = 0;
    pre_s[tid] = 0;
  }
  __syncthreads();
  // Expert totals over all blocks and over the blocks before this one.
  if ((blockDim.x % E) == 0 && (64 % E) == 0) {
    // E divides the block and the wave (a power of two <= 64): every element a
    // thread visits has expert tid % E, so it sums them in registers, the
    // lanes of one expert reduce by shuffles, and each wave adds once per
    // expert (integer sums: order-free).
    int tot = 0, pre = 0;
    for (int i = tid; i < nb * E; i += blockDim.x) {
      const int c = block_counts[i];
      tot += c;
      if (i / E < b) pre += c;
    }
    for (int m = E; m < 64; m <<= 1) {
      tot += __shfl_xor(tot, m);
      pre += __shfl_xor(pre, m);
    }
    if ((tid & 63) < E) {
      atomicAdd(&tot_s[tid & 63], tot);
      atomicAdd(&pre_s[tid & 63], pre);
    }
  } else {
    for (int i = tid; i < nb * E; i += blockDim.x) {
      const int bb = i / E;
      const int ee = i - bb * E;
      const int c = block_counts[i];
      atomicAdd(&tot_s[ee], c);
      if (bb < b) atomicAdd(&pre_s[ee], c);
    }
  }
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int e = 0; e < E; ++e) {
      base_s[e] = run + pre_s[e];
      if (b == 0) offsets[e] = run;
      run += tot_s[e];
    }
    if (b == 0) {
      offsets[E] = run;  // == T * k
      offsets[E + 1] = run + T;
    }
  }
  __syncthreads();
  // Stable placement (place_entries' order), the first window from the
  // registers loaded above.
  if (tid < 64) {
    const int lane = tid;
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    int base = lane < E ? base_s[lane] : 0;  // running base of expert `lane`
    for (size_t ws = s0; ws < s1; ws += 64) {
      const size_t ts = ws + lane;
      const bool live = ts < s1;
      const int e_me = ws == s0 ? e0 : (live ? topk_idx[ts] : -1);
      const float wt = ws == s0 ? w0 : (live ? topk_w[ts] : 0.0f);
      int r = -1;
      for (int e = 0; e < E; ++e) {
        const uint64_t m = __ballot(e_me == e);
        const int be = __shfl(base, e);
        if (e_me == e) r = be + __popcll(m & lt);
        if (lane == e) base += __popcll(m);
      }
      if (live && r >= 0) {
        row_token[r] = (int32_t)(ts / k);
        row_weight[r] = wt;
        token_row[ts] = r;
      }
    }
  }
}

template <typename XT, int LPT, int KC>
int launch_staged_t(const XT *x, const float *w, const float *bias, const float *concept, int nc,
                    int T, int d, int E, int k, float *logits, int32_t *idx, float *wt,
                    int32_t *bc, int nb, hipStream_t s) {
  using Cf = StagedRouter<XT, LPT, KC>;
  static bool attr_set = false;
  if (!attr_set) {
    PRICHS_HIP_TRY(hipFuncSetAttribute(
                       reinterpret_cast<const void *>(&router_topk_staged_kernel<XT, LPT, KC>),
                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)Cf::kLds),
                   "router: set LDS size");
    attr_set = true;
  }
  hipLaunchKernelGGL((router_topk_staged_kernel<XT, LPT, KC>), dim3(nb), dim3(kRouterThreads),
                     Cf::kLds, s, x, w, bias, concept, nc, T, d, E, k, logits, idx, wt, bc);
  return PRICHS_OK;
}

// K chunk per lanes-per-token: both LDS buffers within ~42 KB (three blocks
// per CU) and at most 8 x vectors and 4 W float4s staged per thread.
template <typename XT>
int launch_staged(int lg, const XT *x, const float *w, const float *bias, const float *concept,
                  int nc, int T, int d, int E, int k, float *logits, int32_t *idx, float *wt,
                  int32_t *bc, int nb, hipStream_t s) {
  switch (lg) {
    case 0: return launch_staged_t<XT, 1, 16>(x, w, bias, concept, nc, T, d, E, k, logits, idx, wt, bc, nb, s);
    case 1: return launch_staged_t<XT, 2, 32>(x, w, bias, concept, nc, T, d, E, k, logits, idx, wt, bc, nb, s);
    case 2: return launch_staged_t<XT, 4, 64>(x, w, bias, concept, nc, T, d, E, k, logits, idx, wt, bc, nb, s);
    case 3: return launch_staged_t<XT, 8, 128>(x, w, bias, concept, nc, T, d, E, k, logits, idx, wt, bc, nb, s);
    case 4: return launch_staged_t<XT, 16, 128>(x, w, bias, concept, nc, T, d, E, k, logits, idx, wt, bc, nb, s);
    case 5: return launch_staged_t<XT, 32, 128>(x, w, bias, concept, nc, T, d, E, k, logits, idx, wt, bc, nb, s);
    default: return launch_staged_t<XT, 64, 64>(x, w, bias, concept, nc, T, d, E, k, logits, idx, wt, bc, nb, s);
  }
}

}  // namespace

}  // namespace prichs

using namespace prichs;

extern "C" size_t prichs_router_num_blocks(size_t T, size_t E) {
  if (E == 0 || E > PRICHS_MAX_EXPERTS) return 0;
  const int tpb = kRouterThreads >> lanes_per_token_log2((int)E);
  return cdiv(T, (size_t)tpb);
}

// The router; with perm.offsets set and a batch one workgroup covers, the
// quad kernel also writes the permutation (*fused = true).  w_lds (may be
// null): the router weights already in the quad kernel's LDS layout, W^T
// [E][d + 4] with zero padding.
static int router_topk_impl(const void *x, int x_dtype, const float *w_router,
                            const float *router_bias, const float *concept_bias, size_t n_concept,
                            size_t T, size_t d, size_t E, size_t k, float *logits,
                            int32_t *topk_idx, float *topk_w, int32_t *block_counts, void *stream,
                            FusedPerm perm, bool *fused, const float *w_lds = nullptr) {
  *fused = false;
  PRICHS_REQUIRE(dtype_ok(x_dtype), "router: bad x dtype %d", x_dtype);
  PRICHS_REQUIRE(E >= 1 && E <= PRICHS_MAX_EXPERTS, "router: E=%zu outside [1, %d]", E,
                 PRICHS_MAX_EXPERTS);
  PRICHS_REQUIRE(k >= 1 && k <= E && k <= PRICHS_MAX_TOPK, "router: k=%zu invalid for E=%zu", k,
                 E);
  PRICHS_REQUIRE(d >= 1, "router: d must be positive");
  PRICHS_REQUIRE(T <= (size_t)INT32_MAX / (k + 1) && d <= (size_t)INT32_MAX / 8,
                 "router: T=%zu or d=%zu too large", T, d);
  if (T == 0) return PRICHS_OK;
  PRICHS_REQUIRE(x && w_router && router_bias && topk_idx && topk_w && block_counts,
                 "router: null pointer argument");
  PRICHS_REQUIRE(concept_bias != nullptr || n_concept == 0,
                 "router: concept_bias is NULL but n_concept=%zu", n_concept);
  const int lg = lanes_per_token_log2((int)E);
  const int tpb = kRouterThreads >> lg;
  const int nb = (int)cdiv(T, (size_t)tpb);
  hipStream_t s = as_stream(stream);
  const int nc = (int)(n_concept < E ? n_concept : E);
  const bool staged = (d % 8 == 0) && (reinterpret_cast<uintptr_t>(x) % 16 == 0) &&
                      (reinterpret_cast<uintptr_t>(w_router) % 16 == 0);
  // The quad-broadcast kernel: eight lanes per token, whole 128-wide chunks,
  // and W^T within one CU's LDS.
  const bool quad = staged && lg == 3 && d % 128 == 0 && (size_t)8 * (d + 4) * 4 <= 150 * 1024 &&
                    PRICHS_ROUTER_QUAD;
  if (quad) {
    if (nb != 1 || perm.offsets == nullptr) perm = FusedPerm{nullptr, nullptr, nullptr, nullptr};
    int rc = x_dtype == PRICHS_DTYPE_BF16
                 ? launch_quad_t<bf16_t>(static_cast<const bf16_t *>(x), w_router, router_bias,
                                         concept_bias, nc, (int)T, (int)d, (int)E, (int)k, logits,
                                         topk_idx, topk_w, block_counts, nb, s, perm, w_lds)
                 : launch_quad_t<float>(static_cast<const float *>(x), w_router, router_bias,
                                        concept_bias, nc, (int)T, (int)d, (int)E, (int)k, logits,
                                        topk_idx, topk_w, block_counts, nb, s, perm, w_lds);
    if (rc) return rc;
    *fused = perm.offsets != nullptr;
  } else if (staged) {
    int rc = x_dtype == PRICHS_DTYPE_BF16
                 ? launch_staged<bf16_t>(lg, static_cast<const bf16_t *>(x), w_router,
                                         router_bias, concept_bias, nc, (int)T, (int)d, (int)E,
                                         (int)k, logits, topk_idx, topk_w, block_counts, nb, s)
                 : launch_staged<float>(lg, static_cast<const float *>(x), w_router, router_bias,
                                        concept_bias, nc, (int)T, (int)d, (int)E, (int)k, logits,
                                        topk_idx, topk_w, block_counts, nb, s);
    if (rc) return rc;
  } else {
    const int kc = router_chunk((int)d, (int)E);
    const size_t lds = (size_t)E * (kc + 4) * sizeof(float);
    if (x_dtype == PRICHS_DTYPE_BF16)
      hipLaunchKernelGGL(router_topk_kernel<bf16_t>, dim3(nb), dim3(kRouterThreads), lds, s,
                         static_cast<const bf16_t *>(x), w_router, router_bias, concept_bias, nc,
                         (int)T, (int)d, (int)E, (int)k, lg, kc, logits, topk_idx, topk_w,
                         block_counts);
    else
      hipLaunchKernelGGL(router_topk_kernel<float>, dim3(nb), dim3(kRouterThreads), lds, s,
                         static_cast<const float *>(x), w_router, router_bias, concept_bias, nc,
                         (int)T, (int)d, (int)E, (int)k, lg, kc, logits, topk_idx, topk_w,
                         block_counts);
  }
  PRICHS_LAUNCH_CHECK("router_topk launch");
  return PRICHS_OK;
}

extern "C" int prichs_router_topk(const void *x, int x_dtype, const float *w_router,
                                  const float *router_bias, const float *concept_bias,
                                  size_t n_concept, size_t T, size_t d, size_t E, size_t k,
                                  float *logits, int32_t *topk_idx, float *topk_w,
                                  int32_t *block_counts, void *stream) {
  bool fused;
  return router_topk_impl(x, x_dtype, w_router, router_bias, concept_bias, n_concept, T, d, E, k,
                          logits, topk_idx, topk_w, block_counts, stream,
                          FusedPerm{nullptr, nullptr, nullptr, nullptr}, &fused);
}

namespace prichs {
size_t router_lds_layout_elems(size_t d, size_t E) {
  // The quad kernel's shapes (eight lanes per token, whole 128-wide chunks).
  if (lanes_per_token_log2((int)E) != 3 || d % 128 != 0 || (size_t)8 * (d + 4) * 4 > 150 * 1024)
    return 0;
  return E * (d + 4);
}

void router_lds_layout(const float *w_router, size_t d, size_t E, float *out) {
  for (size_t e = 0; e < E; ++e) {
    for (size_t c = 0; c < d; ++c) out[e * (d + 4) + c] = w_router[c * E + e];
    for (size_t c = d; c < d + 4; ++c) out[e * (d + 4) + c] = 0.0f;
  }
}

int router_topk_lds(const void *x, int x_dtype, const float *w_router, const float *w_lds,
                    const float *router_bias, const float *concept_bias, size_t n_concept,
                    size_t T, size_t d, size_t E, size_t k, float *logits, int32_t *topk_idx,
                    float *topk_w, int32_t *block_counts, void *stream) {
  bool fused;
  return router_topk_impl(x, x_dtype, w_router, router_bias, concept_bias, n_concept, T, d, E, k,
                          logits, topk_idx, topk_w, block_counts, stream,
                          FusedPerm{nullptr, nullptr, nullptr, nullptr}, &fused, w_lds);
}

int router_topk_permute(const void *x, int x_dtype, const float *w_router,
                        const float *router_bias, const float *concept_bias, size_t n_concept,
                        size_t T, size_t d, size_t E, size_t k, float *logits, int32_t *topk_idx,
                        float *topk_w, int32_t *block_counts, int32_t *offsets,
                        int32_t *row_token, float *row_weight, int32_t *token_row,
                        void *stream, const float *w_lds) {
  bool fused = false;
  if (T > 0) {
    PRICHS_REQUIRE(offsets && row_token && row_weight && token_row,
                   "router_permute: null permutation output");
    int rc = router_topk_impl(x, x_dtype, w_router, router_bias, concept_bias, n_concept, T, d, E,
                              k, logits, topk_idx, topk_w, block_counts, stream,
                              FusedPerm{offsets, row_token, row_weight, token_row}, &fused, w_lds);
    if (rc) return rc;
  }
  if (fused) return PRICHS_OK;
  return prichs_permute(topk_idx, topk_w, block_counts, T, E, k, offsets, row_token, row_weight,
                        token_row, stream);
}
}  // namespace prichs

extern "C" int prichs_permute(const int32_t *topk_idx, const float *topk_w,
                              const int32_t *block_counts, size_t T, size_t E, size_t k,
                              int32_t *offsets, int32_t *row_token, float *row_weight,
                              int32_t *token_row, void *stream) {
  PRICHS_REQUIRE(E >= 1 && E <= PRICHS_MAX_EXPERTS, "permute: E=%zu outside [1, %d]", E,
                 PRICHS_MAX_EXPERTS);
  PRICHS_REQUIRE(k >= 1 && k <= E && k <= PRICHS_MAX_TOPK, "permute: k=%zu invalid for E=%zu",
                 k, E);
  PRICHS_REQUIRE(T <= (size_t)INT32_MAX / (k + 1), "permute: T=%zu too large", T);
  PRICHS_REQUIRE(offsets != nullptr, "permute: null offsets");
  hipStream_t s = as_stream(stream);
  if (T == 0) {
    // Empty batch: every group is empty.
    // (A fill kernel rather than hipMemsetAsync, which is unsafe in captured graphs.)
    hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(128), 0, s, offsets, (int)(E + 2), 0);
    PRICHS_LAUNCH_CHECK("permute fill");
    return PRICHS_OK;
  }
  PRICHS_REQUIRE(topk_idx && topk_w && block_counts && row_token && row_weight && token_row,
                 "permute: null pointer argument");
  const int lg = lanes_per_token_log2((int)E);
  const int tpb = kRouterThreads >> lg;
  const int nb = (int)cdiv(T, (size_t)tpb);
  hipLaunchKernelGGL(permute_kernel, dim3(nb), dim3(256), 0, s, topk_idx, topk_w, block_counts,
                     (int)T, (int)E, (int)k, tpb, nb, offsets, row_token, row_weight, token_row);
  PRICHS_LAUNCH_CHECK("permute launch");
  return PRICHS_OK;
}
