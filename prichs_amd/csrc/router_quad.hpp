// router_quad.hpp -- router device code shared by router.hip (the router and
// permutation kernels) and gemm.hip (the decode launch that runs one router
// workgroup beside the gate/up GEMM): top-k gating of one token, the
// permutation of a batch that one workgroup covers, and the body of the
// quad-broadcast router workgroup.  Restates crates/prichs-model/src/
// moe.rs:113-142 and crates/prichs-core/src/ops.rs:219-248 (see router.hip).
#pragma once

#include "common.hpp"

namespace prichs {
namespace rq {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#ifndef PRICHS_ROUTER_THREADS
#define PRICHS_ROUTER_THREADS 256
#endif
constexpr int kRouterThreads = PRICHS_ROUTER_THREADS;  // >= PRICHS_MAX_EXPERTS

// ---------------------------------------------------------------------------
// Top-k gating of one token whose lpt lanes hold (raw, adj) of expert e = lane
// index within the group (crates/prichs-core/src/ops.rs:219-248), then the
// writes of idx / weights and the block's expert histogram.  idx_l / w_l (may
// be null): LDS copies of idx / weights at the same index, for a placement
// by the same workgroup (which then needs no global round trip).
// ---------------------------------------------------------------------------
__device__ inline void topk_epilogue(float acc, float adj, bool valid, int e, int t, int T, int E,
                                     int k, int lpt, float *__restrict__ logits,
                                     int32_t *__restrict__ topk_idx, float *__restrict__ topk_w,
                                     int *cnt_s, int32_t *idx_l = nullptr,
                                     float *w_l = nullptr) {
#pragma clang fp contract(off)
  if (valid && logits != nullptr) logits[(size_t)t * E + e] = acc;

  int nan_any = valid && (adj != adj);
  for (int m = 1; m < lpt; m <<= 1) nan_any |= __shfl_xor(nan_any, m, lpt);

  int sel[PRICHS_MAX_TOPK];
#pragma unroll
  for (int s = 0; s < PRICHS_MAX_TOPK; ++s) sel[s] = 0;

  if (!nan_any) {
    // Stable descending order == order by (adj desc, index asc); +0 == -0.
    bool taken = false;
#pragma unroll
    for (int s = 0; s < PRICHS_MAX_TOPK; ++s) {
      if (s < k) {
        int cv = valid && !taken;
        float cval = adj;
        int cidx = e;
        for (int m = 1; m < lpt; m <<= 1) {
          const int ov = __shfl_xor(cv, m, lpt);
          const float oval = __shfl_xor(cval, m, lpt);
          const int oidx = __shfl_xor(cidx, m, lpt);
          const bool better = ov && (!cv || oval > cval || (oval == cval && oidx < cidx));
          if (better) {
            cv = ov;
            cval = oval;
            cidx = oidx;
          }
        }
        sel[s] = cidx;
        if (cidx == e) taken = true;
      }
    }
  } else {
    // Some adjusted logit is NaN.  The reference's small-slice stable sort is
    // an insertion sort whose comparison (a > b) is false against a NaN, so a
    // NaN never moves and nothing crosses it: the result is each NaN-free
    // segment sorted stably in descending order, NaNs in place.  Position of
    // expert e: its own index if NaN, else segment start + its rank in the
    // segment.
    const bool is_nan = valid && (adj != adj);
    int s0 = 0, s1 = E;
    for (int j = 0; j < lpt; ++j) {
      const float vj = __shfl(adj, j, lpt);
      const bool nj = j < E && (vj != vj);
      if (nj && j < e) s0 = j + 1;
      if (nj && j > e && s1 == E) s1 = j;
    }
    int rank = 0;
    for (int j = 0; j < lpt; ++j) {
      const float vj = __shfl(adj, j, lpt);
      if (j >= s0 && j < s1 && (vj > adj || (vj == adj && j < e))) ++rank;
    }
    const int pos = is_nan ? e : s0 + rank;
#pragma unroll
    for (int s = 0; s < PRICHS_MAX_TOPK; ++s) {
      if (s < k) {
        int who = 0;
        for (int j = 0; j < lpt; ++j) {
          const int pj = __shfl(pos, j, lpt);
          if (j < E && pj == s) who = j;
        }
        sel[s] = who;
      }
    }
  }

  // Softmax over the RAW logits of the selected experts (ops.rs:233-245).
  float rv[PRICHS_MAX_TOPK];
#pragma unroll
  for (int s = 0; s < PRICHS_MAX_TOPK; ++s) rv[s] = (s < k) ? __shfl(acc, sel[s], lpt) : 0.0f;
  float mx = -INFINITY;
#pragma unroll
  for (int s = 0; s < PRICHS_MAX_TOPK; ++s)
    if (s < k) mx = fmaxf(mx, rv[s]);
  float ex[PRICHS_MAX_TOPK];
  float sum = 0.0f;
#pragma unroll
  for (int s = 0; s < PRICHS_MAX_TOPK; ++s) {
    if (s < k) {
      const float diff = rv[s] - mx;
      ex[s] = expf(diff);
      sum = sum + ex[s];
    } else {
      ex[s] = 0.0f;
    }
  }
  const float inv = 1.0f / (sum + 1e-9f);

  if (t < T) {
#pragma unroll
    for (int s = 0; s < PRICHS_MAX_TOPK; ++s) {
      if (s < k && s == e) {
        const float wv = ex[s] * inv;
        topk_idx[(size_t)t * k + s] = sel[s];
        topk_w[(size_t)t * k + s] = wv;
        if (idx_l != nullptr) {
          idx_l[t * k + s] = sel[s];
          w_l[t * k + s] = wv;
        }
        atomicAdd(&cnt_s[sel[s]], 1);  // integer histogram: order-free
      }
    }
  }
}

// Places tokens [t0, t1)'s (token, slot) entries given each expert's first
// row for them (base_s[e]), in (t, s) order, one 64-wide window per wave
// step.  An expert occurs at most once per token, so (t, s) order within one
// expert is token order; each entry's place is the expert's running base
// plus the number of earlier entries of that expert in the window (a ballot
// per expert).  The 64-lane windows are taken in order by wave 0 alone,
// which keeps the running bases sequential.  All threads then write the
// shared-expert rows, which follow the routed rows in token order.
// dense_row (may be null): for each row r of the row space, the row of the
// dense [group][token] layout holding the same (expert, token) pair --
// expert e's row of token t is e * T + t, the shared row of token t is
// E * T + t (the decode path runs the gate/up GEMM densely over all tokens).
__device__ inline void place_entries(const int32_t *__restrict__ topk_idx,
                                     const float *__restrict__ topk_w, int t0, int t1, int T,
                                     int E, int k, const int *base_s, int32_t *__restrict__ row_token,
                                     float *__restrict__ row_weight,
                                     int32_t *__restrict__ token_row,
                                     int32_t *__restrict__ dense_row = nullptr) {
  const int tid = threadIdx.x;
  if (tid < 64) {
    const int lane = tid;
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    int base = lane < E ? base_s[lane] : 0;  // running base of expert `lane`
    const size_t s0 = (size_t)t0 * k, s1 = (size_t)t1 * k;
    for (size_t w0 = s0; w0 < s1; w0 += 64) {
      const size_t ts = w0 + lane;
      const bool live = ts < s1;
      const int e_me = live ? topk_idx[ts] : -1;
      const float wt = live ? topk_w[ts] : 0.0f;
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
        if (dense_row != nullptr) dense_row[r] = e_me * T + (int32_t)(ts / k);
      }
    }
  }
  for (int t = t0 + tid; t < t1; t += blockDim.x) {
    row_token[(size_t)T * k + t] = t;
    if (dense_row != nullptr) dense_row[(size_t)T * k + t] = E * T + t;
  }
}

// Outputs of the permutation, filled by the router's own workgroup when one
// workgroup covers every token (decode-sized batches); offsets == nullptr
// leaves the permutation to permute_kernel.
struct FusedPerm {
  int32_t *offsets, *row_token;
  float *row_weight;
  int32_t *token_row;
  int32_t *dense_row;  // optional (see place_entries)
};

// ---------------------------------------------------------------------------
// Quad-broadcast router (E <= 8, eight lanes per token, d % 128 == 0).  The
// block's router weights sit transposed in LDS for the whole kernel (staged
// once, no barrier in the K loop), and x never goes through LDS: in chunks of
// 128, lane r = e % 4 of each quad loads its quarter (32 values) of the
// token's chunk straight into registers, and every product takes x from the
// quad's holder lane by a DPP quad broadcast folded into the multiply.  Per
// k a lane thus reads 4 bytes of LDS (its expert's weight) instead of 8, and
// at one wave per SIMD nothing waits on a workgroup barrier.  The arithmetic
// is the reference's (k ascending, product rounded, then sum rounded).
// ---------------------------------------------------------------------------
template <typename XT> struct QuadRouter {
  static constexpr int kKC = 128;                 // k per chunk
  static constexpr int kQ = kKC / 4;              // x values a lane holds per chunk
  static constexpr int kVe = 16 / (int)sizeof(XT);
  static constexpr int kLoads = kQ / kVe;         // 16-byte loads per lane per chunk
  static constexpr int kRing = sizeof(XT) == 2 ? 4 : 2;  // chunks in flight
};

// x broadcast from lane h of each quad (quad_perm [h, h, h, h]).
template <int H> __device__ __forceinline__ float quad_bcast(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), H * 0x55, 0xF, 0xF, true));
}

// The body of one router workgroup: tokens [bid * 32, bid * 32 + 32); wt_s
// is the workgroup's LDS for W^T [8][d + 4] (f32, 16-byte aligned).
template <typename XT>
__device__ inline void router_quad_body(
    const XT *__restrict__ x, const float *__restrict__ w, const float *__restrict__ bias,
    const float *__restrict__ concept, int n_concept, int T, int d, int E, int k,
    float *__restrict__ logits, int32_t *__restrict__ topk_idx, float *__restrict__ topk_w,
    int32_t *__restrict__ block_counts, FusedPerm perm, const float *__restrict__ w_lds, int bid,
    float *__restrict__ wt_s) {
#pragma clang fp contract(off)
  using Cf = QuadRouter<XT>;
  constexpr int kTpb = kRouterThreads / 8;
  __shared__ int cnt_s[PRICHS_MAX_EXPERTS];
  const int tid = threadIdx.x;
  const int e = tid & 7, tl = tid >> 3, r = e & 3;
  const int t = bid * kTpb + tl;
  const bool valid = (t < T) && (e < E);
  const int ws = d + 4;
  const int nch = d / Cf::kKC;
  if (tid < E) cnt_s[tid] = 0;

  // This lane's quarter of each chunk (rows past T read row T-1, never summed).
  const XT *xq = x + (size_t)min(t, T - 1) * d + r * Cf::kQ;
  u32x4 ring[Cf::kRing][Cf::kLoads];
  auto fetch = [&](int c, u32x4(&dst)[Cf::kLoads]) {
    const XT *src = xq + (size_t)min(c, nch - 1) * Cf::kKC;
#pragma unroll
    for (int l = 0; l < Cf::kLoads; ++l)
      dst[l] = *reinterpret_cast<const u32x4 *>(src + l * Cf::kVe);
  };
#pragma unroll
  for (int j = 0; j < Cf::kRing; ++j) fetch(j, ring[j]);

  if (w_lds != nullptr) {
    // W^T already in the LDS layout [E][d + 4] (the engine keeps one): a
    // straight copy, up to 16 float4 loads per thread in flight before their
    // stores, so one round trip covers E (d + 4) <= 16384 floats (d = 1536,
    // E = 8: 13 loads per thread; E (d + 4) is a multiple of 4 since
    // d % 128 == 0).
    constexpr int kWB = 16;
    const int n4 = E * ws / 4;
    const f32x4 *src = reinterpret_cast<const f32x4 *>(w_lds);
    f32x4 *dst = reinterpret_cast<f32x4 *>(wt_s);
    for (int base = 0; base < n4; base += kWB * kRouterThreads) {
      f32x4 v[kWB];
#pragma unroll
      for (int u = 0; u < kWB; ++u) v[u] = src[min(base + u * kRouterThreads + tid, n4 - 1)];
#pragma unroll
      for (int u = 0; u < kWB; ++u) {
        const int i = base + u * kRouterThreads + tid;
        if (i < n4) dst[i] = v[u];
      }
    }
  } else {
    // W [d][E] (row-major, the reference layout) -> W^T [e][k] in LDS, in
    // batches of 8 float4 loads per thread issued before their stores (d * E
    // is a multiple of 4 since d % 128 == 0).
    const int n4 = d * E / 4;
    const f32x4 *w4 = reinterpret_cast<const f32x4 *>(w);
    for (int base = 0; base < n4; base += 8 * kRouterThreads) {
      f32x4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = w4[min(base + u * kRouterThreads + tid, n4 - 1)];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int i = base + u * kRouterThreads + tid;
        if (i < n4) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int f = 4 * i + j;  // flat index in [d][E]
            const int kk = E == 8 ? f >> 3 : f / E;
            const int ee = f - kk * E;
            wt_s[ee * ws + kk] = v[u][j];
          }
        }
      }
    }
  }
  __syncthreads();

  const float *wrow = wt_s + (e < E ? e : 0) * ws;
  float acc = 0.0f;
  for (int c0 = 0; c0 < nch; c0 += Cf::kRing) {
#pragma unroll
    for (int j = 0; j < Cf::kRing; ++j) {
      const int c = c0 + j;
      float xf[Cf::kQ];
#pragma unroll
      for (int l = 0; l < Cf::kLoads; ++l) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t u = ring[j][l][q];
          if constexpr (sizeof(XT) == 2) {
            xf[l * 8 + 2 * q] = __uint_as_float(u << 16);
            xf[l * 8 + 2 * q + 1] = __uint_as_float(u & 0xffff0000u);
          } else {
            xf[l * 4 + q] = __uint_as_float(u);
          }
        }
      }
      // Refill on every path (unpredicated) so the compiler's waits stay exact.
      fetch(c + Cf::kRing, ring[j]);
      if (c < nch) {
        const float *wc = wrow + c * Cf::kKC;
        // All of the chunk's weights are read at once (the LDS returns them
        // in order while the sums run), and the products of group g + 1 are
        // formed before the four dependent sums of group g, so each add waits
        // only on the previous add.
        constexpr int kG = Cf::kKC / 4;
        f32x4 wv[kG];
#pragma unroll
        for (int g = 0; g < kG; ++g) wv[g] = *reinterpret_cast<const f32x4 *>(wc + 4 * g);
        auto products = [&](int g, float (&p)[4]) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int kk = 4 * g + q;  // holder lane kk / kQ, its value kk % kQ
            float xv;
            switch (kk / Cf::kQ) {
              case 0: xv = quad_bcast<0>(xf[kk % Cf::kQ]); break;
              case 1: xv = quad_bcast<1>(xf[kk % Cf::kQ]); break;
              case 2: xv = quad_bcast<2>(xf[kk % Cf::kQ]); break;
              default: xv = quad_bcast<3>(xf[kk % Cf::kQ]); break;
            }
            p[q] = xv * wv[g][q];
          }
        };
        float pa[4], pb[4];
        products(0, pa);
#pragma unroll
        for (int g = 0; g < kG; g += 2) {
          if (g + 1 < kG) products(g + 1, pb);
#pragma unroll
          for (int q = 0; q < 4; ++q) acc = acc + pa[q];
          if (g + 2 < kG) products(g + 2, pa);
          if (g + 1 < kG) {
#pragma unroll
            for (int q = 0; q < 4; ++q) acc = acc + pb[q];
          }
        }
      }
    }
  }

  // adj = (raw + bias[e]) (+ concept[e]), moe.rs:126-133.
  float adj = 0.0f;
  if (valid) {
    adj = acc + bias[e];
    if (concept != nullptr && e < n_concept) adj = adj + concept[e];
  }
  // With a fused permutation this is the only workgroup (bid 0, t < kTpb):
  // its selections also go to LDS for the placement below.
  __shared__ int32_t idx_s[kTpb * PRICHS_MAX_TOPK];
  __shared__ float wsel_s[kTpb * PRICHS_MAX_TOPK];
  const bool fused = perm.offsets != nullptr;
  topk_epilogue(acc, adj, valid, e, t, T, E, k, 8, logits, topk_idx, topk_w, cnt_s,
                fused ? idx_s : nullptr, fused ? wsel_s : nullptr);
  __syncthreads();
  if (tid < E) block_counts[(size_t)bid * E + tid] = cnt_s[tid];
  if (fused) {
    // The only workgroup: the histogram is the expert totals, the exclusive
    // scan gives the bases (as permute_kernel's block 0 computes them), and
    // the block's entries (in LDS, visible after the barrier) are placed
    // here.
    __shared__ int base_s[PRICHS_MAX_EXPERTS];
    if (tid == 0) {
      int run = 0;
      for (int ee = 0; ee < E; ++ee) {
        base_s[ee] = run;
        perm.offsets[ee] = run;
        run += cnt_s[ee];
      }
      perm.offsets[E] = run;  // == T * k
      perm.offsets[E + 1] = run + T;
    }
    __syncthreads();
    place_entries(idx_s, wsel_s, 0, T, T, E, k, base_s, perm.row_token, perm.row_weight,
                  perm.token_row, perm.dense_row);
  }
}

}  // namespace rq
}  // namespace prichs
