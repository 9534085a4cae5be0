// elementwise.hip -- HBM-bound kernels: combine, RMSNorm, RoPE, and the
// legacy f32 launchers with the reference's signatures.
//
// All loads/stores are 16-byte vectors along the contiguous dimension where
// the shape allows it (one wave64 sweeps 1 KiB per instruction), with scalar
// fallbacks for ragged shapes.
#include <cmath>
#include <algorithm>

#include "common.hpp"

namespace prichs {
namespace {

// ------------------------------------------------------------- vectors --
struct V8 {
  float v[8];
};

__device__ inline V8 ld8(const float *p) {
  V8 r;
  const float4 a = *reinterpret_cast<const float4 *>(p);
  const float4 b = *reinterpret_cast<const float4 *>(p + 4);
  r.v[0] = a.x; r.v[1] = a.y; r.v[2] = a.z; r.v[3] = a.w;
  r.v[4] = b.x; r.v[5] = b.y; r.v[6] = b.z; r.v[7] = b.w;
  return r;
}
__device__ inline V8 ld8(const bf16_t *p) {
  V8 r;
  const uint4 a = *reinterpret_cast<const uint4 *>(p);
  const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r.v[2 * i] = __uint_as_float(w[i] << 16);
    r.v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
  return r;
}
// ld8 with a non-temporal load (streaming cache policy): for data read for
// the last time, so that it leaves the caches to data that is read again.
typedef uint32_t nt_u32x4 __attribute__((ext_vector_type(4)));
typedef float nt_f32x4 __attribute__((ext_vector_type(4)));
__device__ inline V8 ld8_nt(const float *p) {
  V8 r;
  const nt_f32x4 a = __builtin_nontemporal_load(reinterpret_cast<const nt_f32x4 *>(p));
  const nt_f32x4 b = __builtin_nontemporal_load(reinterpret_cast<const nt_f32x4 *>(p + 4));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r.v[i] = a[i];
    r.v[4 + i] = b[i];
  }
  return r;
}
__device__ inline V8 ld8_nt(const bf16_t *p) {
  V8 r;
  const nt_u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const nt_u32x4 *>(p));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r.v[2 * i] = __uint_as_float(a[i] << 16);
    r.v[2 * i + 1] = __uint_as_float(a[i] & 0xffff0000u);
  }
  return r;
}
template <bool NT, typename T> __device__ inline V8 ld8y(const T *p) {
  if constexpr (NT)
    return ld8_nt(p);
  else
    return ld8(p);
}

__device__ inline void st8(float *p, const V8 &r) {
  *reinterpret_cast<float4 *>(p) = make_float4(r.v[0], r.v[1], r.v[2], r.v[3]);
  *reinterpret_cast<float4 *>(p + 4) = make_float4(r.v[4], r.v[5], r.v[6], r.v[7]);
}
__device__ inline void st8(bf16_t *p, const V8 &r) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = (uint32_t)f32_to_bf16(r.v[2 * i]) | ((uint32_t)f32_to_bf16(r.v[2 * i + 1]) << 16);
  *reinterpret_cast<uint4 *>(p) = make_uint4(w[0], w[1], w[2], w[3]);
}

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

template <typename T> bool aligned16(const T *p) {
  return (reinterpret_cast<uintptr_t>(p) & 15) == 0;
}

// ------------------------------------------------------------- combine --
// out[t] = shared[t] (or 0); then for the token's experts in ascending id:
// out = out + w * y[row]  (crates/prichs-model/src/moe.rs:146, 149, 177-184).
// KC is the top-k as a compile-time constant (the common k = 1, 2 keep the
// index loads and the ordering to a few instructions); KC = 0 takes k at run
// time (k <= PRICHS_MAX_TOPK).  NT: y is read for the last time (see ld8_nt).
template <typename YT, typename OT, bool VEC, int KC, bool NT = false>
__global__ __launch_bounds__(256) void combine_kernel(
    const YT *__restrict__ y, const int32_t *__restrict__ topk_idx,
    const float *__restrict__ topk_w, const int32_t *__restrict__ token_row, int T, int d,
    int k_rt, int has_shared, OT *__restrict__ out) {
#pragma clang fp contract(off)
  constexpr int kMax = KC > 0 ? KC : PRICHS_MAX_TOPK;
  const int k = KC > 0 ? KC : k_rt;
  const int per_tok = VEC ? d / 8 : d;
  const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (long long)T * per_tok) return;
  const int t = (int)(gid / per_tok);
  const int c = (int)(gid - (long long)t * per_tok) * (VEC ? 8 : 1);

  int ex[kMax], rows[kMax];
  float wt[kMax];
#pragma unroll
  for (int s = 0; s < kMax; ++s) {
    if (s < k) {
      ex[s] = topk_idx[(size_t)t * k + s];
      rows[s] = token_row[(size_t)t * k + s];
      wt[s] = topk_w[(size_t)t * k + s];
    } else {
      ex[s] = 0x7fffffff;
      rows[s] = 0;
      wt[s] = 0.f;
    }
  }
  // Ascending expert id: a bubble pass over registers (a single
  // compare-exchange for k = 2).
#pragma unroll
  for (int a = 0; a < kMax - 1; ++a)
#pragma unroll
    for (int b = 0; b < kMax - 1 - a; ++b)
      if (ex[b] > ex[b + 1]) {
        int te = ex[b]; ex[b] = ex[b + 1]; ex[b + 1] = te;
        int tr = rows[b]; rows[b] = rows[b + 1]; rows[b + 1] = tr;
        float tw = wt[b]; wt[b] = wt[b + 1]; wt[b + 1] = tw;
      }

  const size_t shared_row = (size_t)T * k + t;
  if (VEC) {
    V8 acc;
    if (has_shared) {
      acc = ld8y<NT>(y + shared_row * d + c);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) acc.v[j] = 0.f;
    }
#pragma unroll
    for (int s = 0; s < kMax; ++s) {
      if (s < k) {
        const V8 yv = ld8y<NT>(y + (size_t)rows[s] * d + c);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float p = wt[s] * yv.v[j];
          acc.v[j] = acc.v[j] + p;
        }
      }
    }
    st8(out + (size_t)t * d + c, acc);
  } else {
    float acc = has_shared ? Elem<YT>::load(y + shared_row * d + c) : 0.f;
    for (int s = 0; s < k; ++s) {
      const float p = wt[s] * Elem<YT>::load(y + (size_t)rows[s] * d + c);
      acc = acc + p;
    }
    Elem<OT>::store(out + (size_t)t * d + c, acc);
  }
}

// The block's MoE combine followed by its final residual add in one pass
// (crates/prichs-model/src/block.rs:50-68): moe = the combine above (rounded
// to bf16 into moe_out, the sub-layer output), then out = res + moe with res
// the f32 residual x1, rounded to OT -- the arithmetic of combine_kernel
// followed by add_kernel, so both outputs are bit-identical to that pair.
// NT: y is read for the last time (see ld8_nt).
template <typename OT, int KC, bool NT = false>
__global__ __launch_bounds__(256) void combine_residual_kernel(
    const bf16_t *__restrict__ y, const int32_t *__restrict__ topk_idx,
    const float *__restrict__ topk_w, const int32_t *__restrict__ token_row, int T, int d,
    int k_rt, int has_shared, bf16_t *__restrict__ moe_out, const float *__restrict__ res,
    OT *__restrict__ out) {
#pragma clang fp contract(off)
  constexpr int kMax = KC > 0 ? KC : PRICHS_MAX_TOPK;
  const int k = KC > 0 ? KC : k_rt;
  const int per_tok = d / 8;
  const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (long long)T * per_tok) return;
  const int t = (int)(gid / per_tok);
  const int c = (int)(gid - (long long)t * per_tok) * 8;
  int ex[kMax], rows[kMax];
  float wt[kMax];
#pragma unroll
  for (int s = 0; s < kMax; ++s) {
    if (s < k) {
      ex[s] = topk_idx[(size_t)t * k + s];
      rows[s] = token_row[(size_t)t * k + s];
      wt[s] = topk_w[(size_t)t * k + s];
    } else {
      ex[s] = 0x7fffffff;
      rows[s] = 0;
      wt[s] = 0.f;
    }
  }
#pragma unroll
  for (int a = 0; a < kMax - 1; ++a)
#pragma unroll
    for (int b = 0; b < kMax - 1 - a; ++b)
      if (ex[b] > ex[b + 1]) {
        int te = ex[b]; ex[b] = ex[b + 1]; ex[b + 1] = te;
        int tr = rows[b]; rows[b] = rows[b + 1]; rows[b + 1] = tr;
        float tw = wt[b]; wt[b] = wt[b + 1]; wt[b + 1] = tw;
      }
  V8 acc;
  if (has_shared) {
    acc = ld8y<NT>(y + ((size_t)T * k + t) * d + c);
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) acc.v[j] = 0.f;
  }
#pragma unroll
  for (int s = 0; s < kMax; ++s) {
    if (s < k) {
      const V8 yv = ld8y<NT>(y + (size_t)rows[s] * d + c);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float p = wt[s] * yv.v[j];
        acc.v[j] = acc.v[j] + p;
      }
    }
  }
  const size_t o = (size_t)t * d + c;
  st8(moe_out + o, acc);
  const V8 r = ld8(res + o);
  V8 sum;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float m = bf16_to_f32(f32_to_bf16(acc.v[j]));  // the stored (rounded) moe value
    sum.v[j] = r.v[j] + m;
  }
  st8(out + o, sum);
}

// ------------------------------------------------------------- RMSNorm --
// One wave64 per row (crates/prichs-core/src/ops.rs:109-135):
// inv = 1/sqrt(sum(x^2)/d + eps), out = (x * inv) * w.
template <typename XT, typename OT, bool VEC>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const XT *__restrict__ x,
                                                      const float *__restrict__ w,
                                                      OT *__restrict__ out,
                                                      float *__restrict__ rstd, int T, int d,
                                                      float eps) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= T) return;
  const XT *xr = x + (size_t)row * d;
  OT *orow = out + (size_t)row * d;
  float ss = 0.f;
  if (VEC) {
    for (int c = lane * 8; c < d; c += 512) {
      const V8 v = ld8(xr + c);
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = ss + v.v[j] * v.v[j];
    }
  } else {
    for (int c = lane; c < d; c += 64) {
      const float v = Elem<XT>::load(xr + c);
      ss = ss + v * v;
    }
  }
  ss = wave_sum(ss);
  const float rms = sqrtf(ss / (float)d + eps);
  const float inv = 1.0f / rms;
  if (rstd != nullptr && lane == 0) rstd[row] = inv;
  if (VEC) {
    for (int c = lane * 8; c < d; c += 512) {
      V8 v = ld8(xr + c);
      const V8 wv = ld8(w + c);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float a = v.v[j] * inv;
        v.v[j] = a * wv.v[j];
      }
      st8(orow + c, v);
    }
  } else {
    for (int c = lane; c < d; c += 64) {
      const float a = Elem<XT>::load(xr + c) * inv;
      Elem<OT>::store(orow + c, a * w[c]);
    }
  }
}

// RMSNorm of rows with d <= 512 * NCH, each row held in registers between the sum of squares
// and the scaling (one read of x instead of two); the operations and the
// order of the sum are rmsnorm_kernel's vector path, so the results are
// bit-identical to it.
template <typename XT, typename OT, int NCH>
__global__ __launch_bounds__(256) void rmsnorm_reg_kernel(const XT *__restrict__ x,
                                                          const float *__restrict__ w,
                                                          OT *__restrict__ out,
                                                          float *__restrict__ rstd, int T, int d,
                                                          float eps) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= T) return;
  const size_t base = (size_t)row * d;
  V8 v[NCH];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = lane * 8 + 512 * i;
    if (c < d) {
      v[i] = ld8(x + base + c);
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = ss + v[i].v[j] * v[i].v[j];
    }
  }
  ss = wave_sum(ss);
  const float rms = sqrtf(ss / (float)d + eps);
  const float inv = 1.0f / rms;
  if (rstd != nullptr && lane == 0) rstd[row] = inv;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = lane * 8 + 512 * i;
    if (c < d) {
      const V8 wv = ld8(w + c);
      V8 o;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float a = v[i].v[j] * inv;
        o.v[j] = a * wv.v[j];
      }
      st8(out + base + c, o);
    }
  }
}

// ------------------------------------------------- residual add + RMSNorm --
// The block's x1 = x + attn_out (f32) and n2 = rms_norm(x1, w) in one pass
// (crates/prichs-model/src/block.rs:50-68; ops.rs:109-135, 250-267): one wave
// per row keeps its NCH 8-wide chunks of x1 in registers between the sum of
// squares and the scaling.  Every operation, and the order of the sum, is
// that of add_kernel followed by rmsnorm_kernel, so x1 and n2 are
// bit-identical to the two-kernel path.
template <typename A, typename B, int NCH>
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(const A *__restrict__ a,
                                                          const B *__restrict__ b,
                                                          const float *__restrict__ w,
                                                          float *__restrict__ x1,
                                                          bf16_t *__restrict__ out, int T, int d,
                                                          float eps) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= T) return;
  const size_t base = (size_t)row * d;
  V8 v[NCH];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = lane * 8 + 512 * i;
    if (c < d) {
      const V8 va = ld8(a + base + c), vb = ld8(b + base + c);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[i].v[j] = va.v[j] + vb.v[j];
      st8(x1 + base + c, v[i]);
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = ss + v[i].v[j] * v[i].v[j];
    }
  }
  ss = wave_sum(ss);
  const float rms = sqrtf(ss / (float)d + eps);
  const float inv = 1.0f / rms;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = lane * 8 + 512 * i;
    if (c < d) {
      const V8 wv = ld8(w + c);
      V8 o;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float t = v[i].v[j] * inv;
        o.v[j] = t * wv.v[j];
      }
      st8(out + base + c, o);
    }
  }
}

// ---------------------------------------------------------------- RoPE --
// crates/prichs-core/src/backward.rs:160-188: pairs (2i, 2i+1) at position
// p -> (q0 c - q1 s, q0 s + q1 c), c/s = cache[p * hd/2 + i]; sign * s for
// the inverse rotation.  One thread rotates 4 pairs (8 elements).
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void rope_kernel(T *__restrict__ qk, const float *__restrict__ cs,
                                                   const float *__restrict__ sn, long long rows,
                                                   long long ld, int seq_len, int H, int hd,
                                                   int pos_offset, float sign) {
#pragma clang fp contract(off)
  const int half = hd / 2;
  const int per_row = VEC ? half / 4 : half;  // threads per (row, head)
  const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long total = rows * H * per_row;
  if (gid >= total) return;
  const long long rh = gid / per_row;
  const int q = (int)(gid - rh * per_row);
  const long long row = rh / H;
  const int hh = (int)(rh - row * H);
  const int pos = (int)(row % seq_len) + pos_offset;
  T *base = qk + row * ld + (long long)hh * hd;
  const float *cr = cs + (size_t)pos * half;
  const float *sr = sn + (size_t)pos * half;
  if (VEC) {
    const int i0 = q * 4;
    V8 v = ld8(base + 2 * i0);
    const float4 c4 = *reinterpret_cast<const float4 *>(cr + i0);
    const float4 s4 = *reinterpret_cast<const float4 *>(sr + i0);
    const float c[4] = {c4.x, c4.y, c4.z, c4.w};
    const float s[4] = {sign * s4.x, sign * s4.y, sign * s4.z, sign * s4.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float q0 = v.v[2 * j], q1 = v.v[2 * j + 1];
      const float a0 = q0 * c[j], b0 = q1 * s[j];
      const float a1 = q0 * s[j], b1 = q1 * c[j];
      v.v[2 * j] = a0 - b0;
      v.v[2 * j + 1] = a1 + b1;
    }
    st8(base + 2 * i0, v);
  } else {
    const float c = cr[q], s = sign * sr[q];
    const float q0 = Elem<T>::load(base + 2 * q), q1 = Elem<T>::load(base + 2 * q + 1);
    const float a0 = q0 * c, b0 = q1 * s;
    const float a1 = q0 * s, b1 = q1 * c;
    Elem<T>::store(base + 2 * q, a0 - b0);
    Elem<T>::store(base + 2 * q + 1, a1 + b1);
  }
}

// ------------------------------------------------------- legacy kernels --
__global__ __launch_bounds__(256) void swiglu_kernel(const float *__restrict__ g,
                                                     const float *__restrict__ u,
                                                     float *__restrict__ out, size_t n) {
#pragma clang fp contract(off)
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = silu_ref(g[i]) * u[i];
}

__global__ __launch_bounds__(256) void gather_kernel(const float *__restrict__ in,
                                                     const int *__restrict__ idx,
                                                     float *__restrict__ out, size_t n_tok,
                                                     size_t d) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_tok * d) return;
  const size_t r = i / d, c = i - r * d;
  out[i] = in[(size_t)idx[r] * d + c];
}

__global__ __launch_bounds__(256) void scatter_add_kernel(const float *__restrict__ y,
                                                          const int *__restrict__ idx,
                                                          const float *__restrict__ w,
                                                          float *__restrict__ acc, size_t n_tok,
                                                          size_t d) {
#pragma clang fp contract(off)
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_tok * d) return;
  const size_t r = i / d, c = i - r * d;
  const float p = w[r] * y[i];
  atomicAdd(acc + (size_t)idx[r] * d + c, p);
}

unsigned grid_for(size_t n, unsigned block = 256) { return (unsigned)((n + block - 1) / block); }

template <typename XT, typename OT>
void launch_rmsnorm_t(const void *x, const float *w, void *out, float *rstd, size_t T, size_t d,
                      float eps, hipStream_t s) {
  const bool vec = d % 8 == 0 && aligned16(static_cast<const XT *>(x)) &&
                   aligned16(static_cast<OT *>(out)) && aligned16(w);
  auto kern = vec ? rmsnorm_kernel<XT, OT, true> : rmsnorm_kernel<XT, OT, false>;
  if (vec && d <= 1024)
    kern = d <= 512 ? rmsnorm_reg_kernel<XT, OT, 1> : rmsnorm_reg_kernel<XT, OT, 2>;
  else if (vec && d <= 2048)
    kern = d <= 1536 ? rmsnorm_reg_kernel<XT, OT, 3> : rmsnorm_reg_kernel<XT, OT, 4>;
  hipLaunchKernelGGL(kern, dim3((unsigned)cdiv(T, 4)), dim3(256), 0, s,
                     static_cast<const XT *>(x), w, static_cast<OT *>(out), rstd, (int)T, (int)d,
                     eps);
}

template <typename YT, typename OT>
void launch_combine_t(const void *y, const int32_t *idx, const float *w, const int32_t *tr,
                      size_t T, size_t d, size_t k, int has_shared, void *out, hipStream_t s,
                      bool y_last_use) {
  const bool vec =
      d % 8 == 0 && aligned16(static_cast<const YT *>(y)) && aligned16(static_cast<OT *>(out));
  const size_t n = T * (vec ? d / 8 : d);
  auto kern = vec ? (y_last_use ? (k == 2   ? combine_kernel<YT, OT, true, 2, true>
                                   : k == 1 ? combine_kernel<YT, OT, true, 1, true>
                                            : combine_kernel<YT, OT, true, 0, true>)
                                : (k == 2   ? combine_kernel<YT, OT, true, 2>
                                   : k == 1 ? combine_kernel<YT, OT, true, 1>
                                            : combine_kernel<YT, OT, true, 0>))
                  : combine_kernel<YT, OT, false, 0>;
  hipLaunchKernelGGL(kern, dim3(grid_for(n)), dim3(256), 0, s, static_cast<const YT *>(y), idx, w,
                     tr, (int)T, (int)d, (int)k, has_shared, static_cast<OT *>(out));
}

template <typename A, typename B, int NCH>
void launch_add_rmsnorm_nch(const void *a, const void *b, const float *w, float *x1, void *out,
                            size_t T, size_t d, float eps, hipStream_t s) {
  hipLaunchKernelGGL((add_rmsnorm_kernel<A, B, NCH>), dim3((unsigned)cdiv(T, 4)), dim3(256), 0, s,
                     static_cast<const A *>(a), static_cast<const B *>(b), w, x1,
                     static_cast<bf16_t *>(out), (int)T, (int)d, eps);
}

template <typename T>
void launch_rope_t(void *qk, size_t ld, const float *cs, const float *sn, size_t batch, size_t seq,
                   size_t H, size_t hd, size_t pos_off, float sign, hipStream_t s) {
  const size_t half = hd / 2;
  const bool vec = half % 4 == 0 && (ld * sizeof(T)) % 16 == 0 &&
                   aligned16(static_cast<T *>(qk)) && aligned16(cs) && aligned16(sn);
  const long long rows = (long long)(batch * seq);
  const size_t n = (size_t)rows * H * (vec ? half / 4 : half);
  auto kern = vec ? rope_kernel<T, true> : rope_kernel<T, false>;
  hipLaunchKernelGGL(kern, dim3(grid_for(n)), dim3(256), 0, s, static_cast<T *>(qk), cs, sn, rows,
                     (long long)ld, (int)seq, (int)H, (int)hd, (int)pos_off, sign);
}

}  // namespace
}  // namespace prichs

using namespace prichs;

// ------------------------------------------------------------ entry points --
namespace prichs {
int moe_combine(const void *y, int y_dtype, const int32_t *topk_idx, const float *topk_w,
                const int32_t *token_row, size_t T, size_t d, size_t k, int has_shared, void *out,
                int out_dtype, void *stream, bool y_last_use) {
  PRICHS_REQUIRE(dtype_ok(y_dtype) && dtype_ok(out_dtype), "combine: bad dtype");
  PRICHS_REQUIRE(k >= 1 && k <= PRICHS_MAX_TOPK, "combine: k=%zu outside [1, %d]", k,
                 PRICHS_MAX_TOPK);
  PRICHS_REQUIRE(d >= 1 && d <= (size_t)INT32_MAX, "combine: bad d=%zu", d);
  PRICHS_REQUIRE(T <= (size_t)INT32_MAX / (k + 1), "combine: T=%zu too large", T);
  if (T == 0) return PRICHS_OK;
  PRICHS_REQUIRE(y && topk_idx && topk_w && token_row && out, "combine: null pointer argument");
  hipStream_t s = as_stream(stream);
  const int hs = has_shared ? 1 : 0;
  if (y_dtype == PRICHS_DTYPE_BF16) {
    if (out_dtype == PRICHS_DTYPE_BF16)
      launch_combine_t<bf16_t, bf16_t>(y, topk_idx, topk_w, token_row, T, d, k, hs, out, s,
                                        y_last_use);
    else
      launch_combine_t<bf16_t, float>(y, topk_idx, topk_w, token_row, T, d, k, hs, out, s,
                                        y_last_use);
  } else {
    if (out_dtype == PRICHS_DTYPE_BF16)
      launch_combine_t<float, bf16_t>(y, topk_idx, topk_w, token_row, T, d, k, hs, out, s,
                                        y_last_use);
    else
      launch_combine_t<float, float>(y, topk_idx, topk_w, token_row, T, d, k, hs, out, s,
                                        y_last_use);
  }
  PRICHS_LAUNCH_CHECK("combine launch");
  return PRICHS_OK;
}
}  // namespace prichs

extern "C" int prichs_moe_combine(const void *y, int y_dtype, const int32_t *topk_idx,
                                  const float *topk_w, const int32_t *token_row, size_t T,
                                  size_t d, size_t k, int has_shared, void *out, int out_dtype,
                                  void *stream) {
  return moe_combine(y, y_dtype, topk_idx, topk_w, token_row, T, d, k, has_shared, out,
                     out_dtype, stream, false);
}

extern "C" int prichs_rmsnorm_forward(const void *x, int x_dtype, const float *w, void *out,
                                      int out_dtype, float *rstd, size_t T, size_t d, float eps,
                                      void *stream) {
  PRICHS_REQUIRE(dtype_ok(x_dtype) && dtype_ok(out_dtype), "rmsnorm: bad dtype");
  PRICHS_REQUIRE(d >= 1 && d <= (size_t)INT32_MAX && T <= (size_t)INT32_MAX,
                 "rmsnorm: bad shape T=%zu d=%zu", T, d);
  if (T == 0) return PRICHS_OK;
  PRICHS_REQUIRE(x && w && out, "rmsnorm: null pointer argument");
  hipStream_t s = as_stream(stream);
  if (x_dtype == PRICHS_DTYPE_BF16) {
    if (out_dtype == PRICHS_DTYPE_BF16)
      launch_rmsnorm_t<bf16_t, bf16_t>(x, w, out, rstd, T, d, eps, s);
    else
      launch_rmsnorm_t<bf16_t, float>(x, w, out, rstd, T, d, eps, s);
  } else {
    if (out_dtype == PRICHS_DTYPE_BF16)
      launch_rmsnorm_t<float, bf16_t>(x, w, out, rstd, T, d, eps, s);
    else
      launch_rmsnorm_t<float, float>(x, w, out, rstd, T, d, eps, s);
  }
  PRICHS_LAUNCH_CHECK("rmsnorm launch");
  return PRICHS_OK;
}

// RoPE with the sine multiplied by sin_scale (+1 forward, -1 inverse; the
// legacy launcher passes its int backward_sign through, as kernels.cu:543
// does).
static int rope_impl(void *qk, size_t row_stride, int dtype, const float *cos_cache,
                     const float *sin_cache, size_t cache_rows, size_t batch, size_t seq_len,
                     size_t n_heads, size_t head_dim, size_t pos_offset, float sin_scale,
                     void *stream) {
  PRICHS_REQUIRE(dtype_ok(dtype), "rope: bad dtype %d", dtype);
  PRICHS_REQUIRE(head_dim >= 2 && head_dim % 2 == 0, "rope: head_dim=%zu must be even",
                 head_dim);
  PRICHS_REQUIRE(seq_len + pos_offset <= cache_rows,
                 "rope: positions up to %zu exceed the cache (%zu rows)", seq_len + pos_offset,
                 cache_rows);
  PRICHS_REQUIRE(cache_rows <= (size_t)INT32_MAX && n_heads <= (size_t)INT32_MAX,
                 "rope: shape too large");
  PRICHS_REQUIRE(row_stride >= n_heads * head_dim, "rope: row_stride=%zu < n_heads*head_dim",
                 row_stride);
  if (batch == 0 || seq_len == 0 || n_heads == 0) return PRICHS_OK;
  PRICHS_REQUIRE(qk && cos_cache && sin_cache, "rope: null pointer argument");
  hipStream_t s = as_stream(stream);
  if (dtype == PRICHS_DTYPE_BF16)
    launch_rope_t<bf16_t>(qk, row_stride, cos_cache, sin_cache, batch, seq_len, n_heads,
                          head_dim, pos_offset, sin_scale, s);
  else
    launch_rope_t<float>(qk, row_stride, cos_cache, sin_cache, batch, seq_len, n_heads, head_dim,
                         pos_offset, sin_scale, s);
  PRICHS_LAUNCH_CHECK("rope launch");
  return PRICHS_OK;
}

extern "C" int prichs_rope_forward_ld(void *qk, size_t row_stride, int dtype,
                                      const float *cos_cache, const float *sin_cache,
                                      size_t cache_rows, size_t batch, size_t seq_len,
                                      size_t n_heads, size_t head_dim, size_t pos_offset, int sign,
                                      void *stream) {
  PRICHS_REQUIRE(sign == 1 || sign == -1, "rope: sign must be +1 or -1");
  return rope_impl(qk, row_stride, dtype, cos_cache, sin_cache, cache_rows, batch, seq_len,
                   n_heads, head_dim, pos_offset, (float)sign, stream);
}

extern "C" int prichs_rope_forward(void *qk, int dtype, const float *cos_cache,
                                   const float *sin_cache, size_t cache_rows, size_t batch,
                                   size_t seq_len, size_t n_heads, size_t head_dim,
                                   size_t pos_offset, int sign, void *stream) {
  return prichs_rope_forward_ld(qk, n_heads * head_dim, dtype, cos_cache, sin_cache, cache_rows,
                                batch, seq_len, n_heads, head_dim, pos_offset, sign, stream);
}

// out = a + b element-wise (crates/prichs-core/src/ops.rs:250-267), f32
// arithmetic, operands and result each bf16 or f32.
template <typename A, typename B, typename O>
__global__ __launch_bounds__(256) void add_kernel(const A *__restrict__ a, const B *__restrict__ b,
                                                  O *__restrict__ out, long long n8) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n8) return;
  const V8 va = ld8(a + 8 * i), vb = ld8(b + 8 * i);
  V8 r;
#pragma unroll
  for (int j = 0; j < 8; ++j) r.v[j] = va.v[j] + vb.v[j];
  st8(out + 8 * i, r);
}

template <typename A, typename B, typename O>
void launch_add_t(const void *a, const void *b, void *out, size_t n, hipStream_t s) {
  const long long n8 = (long long)(n / 8);
  hipLaunchKernelGGL((add_kernel<A, B, O>), dim3(grid_for((size_t)n8)), dim3(256), 0, s,
                     static_cast<const A *>(a), static_cast<const B *>(b), static_cast<O *>(out),
                     n8);
}

namespace prichs {
// x1 = a + b (f32) and out = rms_norm(x1, w) (bf16) in one kernel when every
// row fits the register chunks (d % 8 == 0, d <= 2048, 16-byte aligned);
// otherwise prichs_add then prichs_rmsnorm_forward.  Same results either way.
int add_rmsnorm_forward(const void *a, int a_dtype, const void *b, int b_dtype, float *x1,
                        const float *w, void *out, size_t T, size_t d, float eps, void *stream) {
  PRICHS_REQUIRE(dtype_ok(a_dtype) && dtype_ok(b_dtype), "add_rmsnorm: bad dtype");
  if (T == 0) return PRICHS_OK;
  PRICHS_REQUIRE(a && b && x1 && w && out, "add_rmsnorm: null pointer argument");
  const bool fused = d % 8 == 0 && d <= 2048 &&
                     ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
                       reinterpret_cast<uintptr_t>(x1) | reinterpret_cast<uintptr_t>(w) |
                       reinterpret_cast<uintptr_t>(out)) & 15) == 0 &&
                     a_dtype == PRICHS_DTYPE_BF16 && b_dtype == PRICHS_DTYPE_BF16;
  if (!fused) {
    int rc = prichs_add(a, a_dtype, b, b_dtype, x1, PRICHS_DTYPE_F32, T * d, stream);
    if (rc) return rc;
    return prichs_rmsnorm_forward(x1, PRICHS_DTYPE_F32, w, out, PRICHS_DTYPE_BF16, nullptr, T, d,
                                  eps, stream);
  }
  hipStream_t s = as_stream(stream);
  const size_t nch = cdiv(d, (size_t)512);
  if (nch <= 1)
    launch_add_rmsnorm_nch<bf16_t, bf16_t, 1>(a, b, w, x1, out, T, d, eps, s);
  else if (nch == 2)
    launch_add_rmsnorm_nch<bf16_t, bf16_t, 2>(a, b, w, x1, out, T, d, eps, s);
  else if (nch == 3)
    launch_add_rmsnorm_nch<bf16_t, bf16_t, 3>(a, b, w, x1, out, T, d, eps, s);
  else
    launch_add_rmsnorm_nch<bf16_t, bf16_t, 4>(a, b, w, x1, out, T, d, eps, s);
  PRICHS_LAUNCH_CHECK("add_rmsnorm launch");
  return PRICHS_OK;
}
}  // namespace prichs

namespace prichs {
// moe_out = combine (bf16) and out = res + moe_out in one kernel when the
// vector path applies (bf16 y, d % 8 == 0, 16-byte aligned); otherwise
// prichs_moe_combine then prichs_add.  Same results either way.
int moe_combine_residual(const void *y, const int32_t *topk_idx, const float *topk_w,
                         const int32_t *token_row, size_t T, size_t d, size_t k, int has_shared,
                         void *moe_out, const float *res, void *out, int out_dtype,
                         void *stream, bool y_last_use) {
  PRICHS_REQUIRE(dtype_ok(out_dtype), "combine_residual: bad out dtype");
  PRICHS_REQUIRE(k >= 1 && k <= PRICHS_MAX_TOPK, "combine_residual: bad k=%zu", k);
  if (T == 0) return PRICHS_OK;
  PRICHS_REQUIRE(y && topk_idx && topk_w && token_row && moe_out && res && out,
                 "combine_residual: null pointer argument");
  const bool fused = d % 8 == 0 &&
                     ((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(moe_out) |
                       reinterpret_cast<uintptr_t>(res) | reinterpret_cast<uintptr_t>(out)) & 15) == 0;
  if (!fused) {
    int rc = moe_combine(y, PRICHS_DTYPE_BF16, topk_idx, topk_w, token_row, T, d, k, has_shared,
                         moe_out, PRICHS_DTYPE_BF16, stream, y_last_use);
    if (rc) return rc;
    return prichs_add(res, PRICHS_DTYPE_F32, moe_out, PRICHS_DTYPE_BF16, out, out_dtype, T * d,
                      stream);
  }
  hipStream_t s = as_stream(stream);
  const unsigned grid = grid_for(T * (d / 8));
#define PRICHS_COMBINE_RES(OT_, KC_, NT_)                                                     \
  hipLaunchKernelGGL((combine_residual_kernel<OT_, KC_, NT_>), dim3(grid), dim3(256), 0, s,   \
                     static_cast<const bf16_t *>(y), topk_idx, topk_w, token_row, (int)T,     \
                     (int)d, (int)k, has_shared, static_cast<bf16_t *>(moe_out), res,         \
                     static_cast<OT_ *>(out))
  if (out_dtype == PRICHS_DTYPE_BF16) {
    if (k == 2) {
      if (y_last_use)
        PRICHS_COMBINE_RES(bf16_t, 2, true);
      else
        PRICHS_COMBINE_RES(bf16_t, 2, false);
    } else {
      PRICHS_COMBINE_RES(bf16_t, 0, false);
    }
  } else {
    if (k == 2) {
      if (y_last_use)
        PRICHS_COMBINE_RES(float, 2, true);
      else
        PRICHS_COMBINE_RES(float, 2, false);
    } else {
      PRICHS_COMBINE_RES(float, 0, false);
    }
  }
#undef PRICHS_COMBINE_RES
  PRICHS_LAUNCH_CHECK("combine_residual launch");
  return PRICHS_OK;
}
}  // namespace prichs

extern "C" int prichs_add(const void *a, int a_dtype, const void *b, int b_dtype, void *out,
                          int out_dtype, size_t n, void *stream) {
  PRICHS_REQUIRE(dtype_ok(a_dtype) && dtype_ok(b_dtype) && dtype_ok(out_dtype), "add: bad dtype");
  PRICHS_REQUIRE(n % 8 == 0, "add: n=%zu must be a multiple of 8", n);
  if (n == 0) return PRICHS_OK;
  PRICHS_REQUIRE(a && b && out, "add: null pointer argument");
  PRICHS_REQUIRE(((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
                   reinterpret_cast<uintptr_t>(out)) & 15) == 0,
                 "add: operands must be 16-byte aligned");
  hipStream_t s = as_stream(stream);
  const int key = a_dtype * 4 + b_dtype * 2 + out_dtype;
  switch (key) {
    case 0: launch_add_t<float, float, float>(a, b, out, n, s); break;
    case 1: launch_add_t<float, float, bf16_t>(a, b, out, n, s); break;
    case 2: launch_add_t<float, bf16_t, float>(a, b, out, n, s); break;
    case 3: launch_add_t<float, bf16_t, bf16_t>(a, b, out, n, s); break;
    case 4: launch_add_t<bf16_t, float, float>(a, b, out, n, s); break;
    case 5: launch_add_t<bf16_t, float, bf16_t>(a, b, out, n, s); break;
    case 6: launch_add_t<bf16_t, bf16_t, float>(a, b, out, n, s); break;
    default: launch_add_t<bf16_t, bf16_t, bf16_t>(a, b, out, n, s); break;
  }
  PRICHS_LAUNCH_CHECK("add launch");
  return PRICHS_OK;
}

// RoPE tables on the host (crates/prichs-core/src/backward.rs:136-157):
// freq_i = 1 / theta^((2i)/hd) with libm powf, angle = (t as f32) * freq_i,
// cos/sin with libm cosf/sinf -- the functions Rust's f32 methods call.
extern "C" int prichs_rope_cache(size_t max_seq_len, size_t head_dim, float theta,
                                 float *cos_out, float *sin_out) {
  PRICHS_REQUIRE(head_dim >= 2 && head_dim % 2 == 0, "rope_cache: head_dim=%zu must be even",
                 head_dim);
  PRICHS_REQUIRE(cos_out && sin_out, "rope_cache: null pointer argument");
  PRICHS_REQUIRE(max_seq_len <= ((size_t)1 << 31), "rope_cache: max_seq_len too large");
  const size_t half = head_dim / 2;
  for (size_t i = 0; i < half; ++i) {
    volatile float exponent = (float)(2 * i) / (float)head_dim;
    const float freq = 1.0f / powf(theta, exponent);
    for (size_t t = 0; t < max_seq_len; ++t) {
      volatile float angle = (float)t * freq;
      cos_out[t * half + i] = cosf(angle);
      sin_out[t * half + i] = sinf(angle);
    }
  }
  return PRICHS_OK;
}

// ---------------------------------------------------------- legacy ABI --
// void launchers: failures go to the last-error slot only, like the
// reference's unchecked launchers.
extern "C" void launch_rmsnorm_forward(const float *dev_x, const float *dev_weight, float *dev_out,
                                       float *dev_rstd_out, size_t seq_len, size_t hidden_dim,
                                       float eps, void *stream) {
  (void)prichs_rmsnorm_forward(dev_x, PRICHS_DTYPE_F32, dev_weight, dev_out, PRICHS_DTYPE_F32,
                               dev_rstd_out, seq_len, hidden_dim, eps, stream);
}

extern "C" void launch_swiglu_forward(const float *dev_gate, const float *dev_up, float *dev_out,
                                      size_t total_elements, void *stream) {
  if (total_elements == 0) return;
  if (!dev_gate || !dev_up || !dev_out) {
    set_error("launch_swiglu_forward: null pointer argument");
    return;
  }
  hipLaunchKernelGGL(swiglu_kernel, dim3(grid_for(total_elements)), dim3(256), 0,
                     as_stream(stream), dev_gate, dev_up, dev_out, total_elements);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) set_error("launch_swiglu_forward: %s", hipGetErrorString(e));
}

extern "C" void launch_rope(float *dev_q_or_k, const float *dev_cos_cache,
                            const float *dev_sin_cache, size_t seq_len, size_t num_heads,
                            size_t head_dim, int backward_sign, void *stream) {
  // sin * (float)backward_sign, whatever the int (kernels.cu:543).
  (void)rope_impl(dev_q_or_k, num_heads * head_dim, PRICHS_DTYPE_F32, dev_cos_cache,
                  dev_sin_cache, seq_len, 1, seq_len, num_heads, head_dim, 0,
                  (float)backward_sign, stream);
}

extern "C" void launch_moe_gather(const float *dev_in, const int *dev_token_indices,
                                  float *dev_out, size_t n_tokens, size_t hidden_dim,
                                  void *stream) {
  const size_t n = n_tokens * hidden_dim;
  if (n == 0) return;
  if (!dev_in || !dev_token_indices || !dev_out) {
    set_error("launch_moe_gather: null pointer argument");
    return;
  }
  hipLaunchKernelGGL(gather_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), dev_in,
                     dev_token_indices, dev_out, n_tokens, hidden_dim);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) set_error("launch_moe_gather: %s", hipGetErrorString(e));
}

extern "C" void launch_moe_scatter_add(const float *dev_exp_out, const int *dev_token_indices,
                                       const float *dev_weights, float *dev_accum_out,
                                       size_t n_tokens, size_t hidden_dim, void *stream) {
  const size_t n = n_tokens * hidden_dim;
  if (n == 0) return;
  if (!dev_exp_out || !dev_token_indices || !dev_weights || !dev_accum_out) {
    set_error("launch_moe_scatter_add: null pointer argument");
    return;
  }
  hipLaunchKernelGGL(scatter_add_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream),
                     dev_exp_out, dev_token_indices, dev_weights, dev_accum_out, n_tokens,
                     hidden_dim);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) set_error("launch_moe_scatter_add: %s", hipGetErrorString(e));
}

// ------------------------------------------------------------------------
// Streaming device copy: the build's own practical HBM yardstick for the
// memory-bound stages (what a plain 16-byte-per-lane kernel moves on this
// chip), timed like them.  Each thread loads kCopyUnroll 16-byte chunks of a
// workgroup block (consecutive lanes, consecutive chunks: every wave
// instruction covers 1 KiB contiguous), then stores them; workgroups stride
// over the buffer block by block.
// ------------------------------------------------------------------------
namespace prichs {
namespace {
typedef uint32_t cp_u32x4 __attribute__((ext_vector_type(4)));
constexpr int kCopyThreads = 256, kCopyUnroll = 8;

__global__ __launch_bounds__(kCopyThreads) void hbm_copy_kernel(const cp_u32x4 *__restrict__ src,
                                                                cp_u32x4 *__restrict__ dst,
                                                                size_t n16) {
  constexpr size_t kBlock = (size_t)kCopyThreads * kCopyUnroll;
  for (size_t base = (size_t)blockIdx.x * kBlock; base < n16; base += (size_t)gridDim.x * kBlock) {
    const size_t i0 = base + threadIdx.x;
    if (base + kBlock <= n16) {
      cp_u32x4 v[kCopyUnroll];
#pragma unroll
      for (int u = 0; u < kCopyUnroll; ++u) v[u] = src[i0 + (size_t)u * kCopyThreads];
#pragma unroll
      for (int u = 0; u < kCopyUnroll; ++u) dst[i0 + (size_t)u * kCopyThreads] = v[u];
    } else {
      for (int u = 0; u < kCopyUnroll; ++u) {
        const size_t i = i0 + (size_t)u * kCopyThreads;
        if (i < n16) dst[i] = src[i];
      }
    }
  }
}
}  // namespace
}  // namespace prichs

extern "C" int prichs_hbm_copy(const void *src, void *dst, size_t bytes, void *stream) {
  PRICHS_REQUIRE(bytes % 16 == 0, "hbm_copy: bytes=%zu must be a multiple of 16", bytes);
  if (bytes == 0) return PRICHS_OK;
  PRICHS_REQUIRE(src && dst, "hbm_copy: null pointer argument");
  PRICHS_REQUIRE(((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0,
                 "hbm_copy: src and dst must be 16-byte aligned");
  const uintptr_t s0 = reinterpret_cast<uintptr_t>(src), d0 = reinterpret_cast<uintptr_t>(dst);
  PRICHS_REQUIRE(s0 + bytes <= d0 || d0 + bytes <= s0, "hbm_copy: src and dst overlap");
  const int cus = device_cu_count();
  if (cus <= 0) return fail(PRICHS_ERR_HIP, "hbm_copy: cannot query the device");
  const size_t n16 = bytes / 16;
  const size_t blocks = (n16 + (size_t)kCopyThreads * kCopyUnroll - 1) / ((size_t)kCopyThreads * kCopyUnroll);
  const unsigned grid = (unsigned)std::min<size_t>(blocks, (size_t)cus * 8);
  hipLaunchKernelGGL(hbm_copy_kernel, dim3(grid), dim3(kCopyThreads), 0, as_stream(stream),
                     static_cast<const cp_u32x4 *>(src), static_cast<cp_u32x4 *>(dst), n16);
  PRICHS_LAUNCH_CHECK("hbm_copy launch");
  return PRICHS_OK;
}
