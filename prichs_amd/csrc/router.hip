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

namespace prichs {

namespace {

constexpr int kRouterThreads = 256;
constexpr int kRouterLdsBytes = 60 * 1024;

int lanes_per_token_log2(int E) {
  int l = 0;
  while ((1 << l) < E) ++l;
  return l;
}

// Width of the router-weight chunk held in LDS as [E][kc + 4] f32.
int router_chunk(int d, int E) {
  int kc = (kRouterLdsBytes / 4) / E - 4;
  kc = kc / 8 * 8;
  int dpad = (d + 7) / 8 * 8;
  return kc < dpad ? kc : dpad;
}

__device__ inline void load8(const float *p, float *v) {
  const float4 a = *reinterpret_cast<const float4 *>(p);
  const float4 b = *reinterpret_cast<const float4 *>(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

__device__ inline void load8(const bf16_t *p, float *v) {
  const uint4 a = *reinterpret_cast<const uint4 *>(p);
  const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(w[i] << 16);
    v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

template <typename XT, bool VEC>
__global__ __launch_bounds__(kRouterThreads) void router_topk_kernel(
    const XT *__restrict__ x, const float *__restrict__ w,
    const float *__restrict__ bias, const float *__restrict__ concept,
    int n_concept, int T, int d, int E, int k, int lpt_log2, int kc,
    float *__restrict__ logits, int32_t *__restrict__ topk_idx,
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

  // raw[t, e] = sum over k ascending of x[t, k] * W[k, e] (mul, then add).
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
      int kk = 0;
      if (VEC) {
        for (; kk + 8 <= n; kk += 8) {
          float xv[8];
          load8(xr + kk, xv);
          const float4 w0 = *reinterpret_cast<const float4 *>(wr + kk);
          const float4 w1 = *reinterpret_cast<const float4 *>(wr + kk + 4);
          const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float p = xv[j] * wv[j];
            acc = acc + p;
          }
        }
      }
      for (; kk < n; ++kk) {
        const float p = Elem<XT>::load(xr + kk) * wr[kk];
        acc = acc + p;
      }
    }
  }

  // adj = (raw + bias[e]) (+ concept[e]), moe.rs:126-133.
  float adj = 0.0f;
  if (valid) {
    adj = acc + bias[e];
    if (concept != nullptr && e < n_concept) adj = adj + concept[e];
    if (logits != nullptr) logits[(size_t)t * E + e] = acc;
  }

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
          const bool better =
              ov && (!cv || oval > cval || (oval == cval && oidx < cidx));
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
    // Some adjusted logit is NaN: replay the reference's small-slice stable
    // sort (insertion sort, is_less(a, b) == a > b) on the group's values.
    float vals[PRICHS_MAX_EXPERTS];
    int ord[PRICHS_MAX_EXPERTS];
    for (int i = 0; i < E; ++i) {
      vals[i] = __shfl(adj, i, lpt);
      ord[i] = i;
    }
    for (int i = 1; i < E; ++i) {
      const float vi = vals[i];
      const int oi = ord[i];
      int j = i;
      while (j > 0 && vi > vals[j - 1]) {
        vals[j] = vals[j - 1];
        ord[j] = ord[j - 1];
        --j;
      }
      vals[j] = vi;
      ord[j] = oi;
    }
#pragma unroll
    for (int s = 0; s < PRICHS_MAX_TOPK; ++s)
      if (s < k) sel[s] = ord[s];
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
        topk_idx[(size_t)t * k + s] = sel[s];
        topk_w[(size_t)t * k + s] = ex[s] * inv;
        atomicAdd(&cnt_s[sel[s]], 1);  // integer histogram: order-free
      }
    }
  }
  __syncthreads();
  if (tid < E) block_counts[(size_t)blockIdx.x * E + tid] = cnt_s[tid];
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
  if (tid < E) {
    tot_s[tid] = 0;
    pre_s[tid] = 0;
  }
  __syncthreads();
  // Expert totals over all blocks and over the blocks before this one.
  for (int i = tid; i < nb * E; i += blockDim.x) {
    const int bb = i / E;
    const int ee = i - bb * E;
    const int c = block_counts[i];
    atomicAdd(&tot_s[ee], c);
    if (bb < b) atomicAdd(&pre_s[ee], c);
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
  const int t0 = b * tpb;
  const int t1 = min(T, t0 + tpb);
  if (tid < E) {
    int r = base_s[tid];
    for (int t = t0; t < t1; ++t) {
      for (int s = 0; s < k; ++s) {
        const size_t ts = (size_t)t * k + s;
        if (topk_idx[ts] == tid) {
          row_token[r] = t;
          row_weight[r] = topk_w[ts];
          token_row[ts] = r;
          ++r;
        }
      }
    }
  }
  // Shared-expert rows follow the routed rows in token order.
  for (int t = t0 + tid; t < t1; t += blockDim.x) row_token[(size_t)T * k + t] = t;
}

}  // namespace

}  // namespace prichs

using namespace prichs;

extern "C" size_t prichs_router_num_blocks(size_t T, size_t E) {
  if (E == 0 || E > PRICHS_MAX_EXPERTS) return 0;
  const int tpb = kRouterThreads >> lanes_per_token_log2((int)E);
  return cdiv(T, (size_t)tpb);
}

extern "C" int prichs_router_topk(const void *x, int x_dtype, const float *w_router,
                                  const float *router_bias, const float *concept_bias,
                                  size_t n_concept, size_t T, size_t d, size_t E, size_t k,
                                  float *logits, int32_t *topk_idx, float *topk_w,
                                  int32_t *block_counts, void *stream) {
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
  const int kc = router_chunk((int)d, (int)E);
  const size_t lds = (size_t)E * (kc + 4) * sizeof(float);
  const bool vec = (d % 8 == 0) && (reinterpret_cast<uintptr_t>(x) % 16 == 0);
  hipStream_t s = as_stream(stream);
  const int nc = (int)(n_concept < E ? n_concept : E);
  if (x_dtype == PRICHS_DTYPE_BF16) {
    auto kern = vec ? router_topk_kernel<bf16_t, true> : router_topk_kernel<bf16_t, false>;
    hipLaunchKernelGGL(kern, dim3(nb), dim3(kRouterThreads), lds, s,
                       static_cast<const bf16_t *>(x), w_router, router_bias, concept_bias, nc,
                       (int)T, (int)d, (int)E, (int)k, lg, kc, logits, topk_idx, topk_w,
                       block_counts);
  } else {
    auto kern = vec ? router_topk_kernel<float, true> : router_topk_kernel<float, false>;
    hipLaunchKernelGGL(kern, dim3(nb), dim3(kRouterThreads), lds, s,
                       static_cast<const float *>(x), w_router, router_bias, concept_bias, nc,
                       (int)T, (int)d, (int)E, (int)k, lg, kc, logits, topk_idx, topk_w,
                       block_counts);
  }
  PRICHS_LAUNCH_CHECK("router_topk launch");
  return PRICHS_OK;
}

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
    PRICHS_HIP_TRY(hipMemsetAsync(offsets, 0, sizeof(int32_t) * (E + 2), s), "permute memset");
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
