// common.hpp -- shared helpers of libprichs_hip.so (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "prichs_hip.h"

namespace prichs {

// ---------------------------------------------------------------- errors --
void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));

// Returns `code` after recording the message (for `return fail(...)`).
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

// Checks a HIP call; on failure records "<what>: <hip error>" and returns
// PRICHS_ERR_HIP from the enclosing int function.
#define PRICHS_HIP_TRY(expr, what)                                            \
  do {                                                                         \
    hipError_t _e = (expr);                                                    \
    if (_e != hipSuccess)                                                      \
      return ::prichs::fail(PRICHS_ERR_HIP, "%s: %s", (what),                 \
                            hipGetErrorString(_e));                            \
  } while (0)

// After a kernel launch: reports launch-configuration errors.
#define PRICHS_LAUNCH_CHECK(what) PRICHS_HIP_TRY(hipGetLastError(), (what))

#define PRICHS_REQUIRE(cond, ...)                                              \
  do {                                                                         \
    if (!(cond)) return ::prichs::fail(PRICHS_ERR_INVALID_ARGUMENT, __VA_ARGS__); \
  } while (0)

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// Number of compute units of the current device (cached per device).
int device_cu_count();

// ------------------------------------------------------------------ bf16 --
typedef uint16_t bf16_t;

__host__ __device__ inline float bf16_to_f32(bf16_t b) {
  union {
    uint32_t u;
    float f;
  } v;
  v.u = static_cast<uint32_t>(b) << 16;
  return v.f;
}

// Round to nearest even; NaN stays a (quiet) NaN.
__host__ __device__ inline bf16_t f32_to_bf16(float f) {
  union {
    uint32_t u;
    float f;
  } v;
  v.f = f;
  uint32_t u = v.u;
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu))
    return static_cast<bf16_t>((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<bf16_t>(u >> 16);
}

template <typename T> struct Elem;
template <> struct Elem<float> {
  static constexpr int dtype = PRICHS_DTYPE_F32;
  __device__ static float load(const float *p) { return *p; }
  __device__ static void store(float *p, float v) { *p = v; }
};
template <> struct Elem<bf16_t> {
  static constexpr int dtype = PRICHS_DTYPE_BF16;
  __device__ static float load(const bf16_t *p) { return bf16_to_f32(*p); }
  __device__ static void store(bf16_t *p, float v) { *p = f32_to_bf16(v); }
};

inline size_t dtype_size(int dtype) { return dtype == PRICHS_DTYPE_BF16 ? 2 : 4; }
inline bool dtype_ok(int dtype) {
  return dtype == PRICHS_DTYPE_F32 || dtype == PRICHS_DTYPE_BF16;
}

inline size_t roundup(size_t a, size_t b) { return (a + b - 1) / b * b; }
inline size_t cdiv(size_t a, size_t b) { return (a + b - 1) / b; }

// Device-side silu of the reference CPU path (crates/prichs-core/src/ops.rs:
// 137-140): x / (1 + exp(-x)).
__device__ inline float silu_ref(float x) { return x / (1.0f + expf(-x)); }

// silu(x) = x / (1 + exp(-x)) on the hardware transcendental units:
// exp(-x) = 2^(-x log2 e) with v_exp_f32, then v_rcp_f32 (each about 1 ulp).
// The result stays within a few ulp of silu_ref, far inside the bf16 bar;
// used by the bf16 GEMM epilogue, whose output is rounded to bf16 anyway.
__device__ inline float silu_fast(float x) {
  const float e = __builtin_amdgcn_exp2f(x * -1.44269504088896341f);
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

// Two floats -> two bf16 (round to nearest even) packed low/high in 32 bits:
// one v_cvt_pk_bf16_f32 (the software f32_to_bf16 agrees on every non-NaN).
typedef float prichs_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 prichs_bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const prichs_f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, prichs_bf16x2));
}

// SwiGLU backward of one element (kernels.cu:459-480): sig = 1 / (1 + exp(-g)),
// silu = g sig, dsilu = sig (1 + g (1 - sig)), dU = dA silu, dG = (dA u)
// dsilu, each operation rounded on its own.  Shared by the SwiGLU backward
// kernel and the dA GEMM epilogue that fuses it, so both give the same bits.
__device__ __forceinline__ void swiglu_bwd_elem(float g, float u, float a, float &dg, float &du) {
#pragma clang fp contract(off)
  const float sig = 1.0f / (1.0f + expf(-g));
  const float silu = g * sig;
  const float dsilu = sig * (1.0f + g * (1.0f - sig));
  du = a * silu;
  const float au = a * u;
  dg = au * dsilu;
}

// prichs_grouped_gate_up_swiglu / prichs_grouped_down with a tighter bound on
// every group's row count (a caller that knows T passes T): decode-sized
// groups then take the skinny weight-streaming kernel.  pre (may be null)
// also receives the gate/up pre-activations [rows][Np] in the packed column
// order (Np = prichs_packed_gate_up_elems(1, f, dtype)), for a backward.
int grouped_gate_up_swiglu_rows(const void *x, const int32_t *row_token, const int32_t *offsets,
                                size_t G, size_t max_rows, size_t max_group_rows,
                                const void *w_packed, size_t d, size_t f, int dtype, void *act,
                                void *stream, void *pre = nullptr);
int grouped_down_rows(const void *act, const int32_t *offsets, size_t G, size_t max_rows,
                      size_t max_group_rows, const void *w_packed, size_t d, size_t f, int dtype,
                      void *y, void *stream);

// Decode path (gemm.hip).  When one router workgroup covers the batch, every
// expert's weights are streamed whatever the routing, so one launch runs the
// router (which also writes the permutation) in its first workgroup while the
// others run the gate/up GEMM densely over all T tokens of every group:
// act_dense [(E + 1) T][f], group g's rows g T .. g T + T - 1 (routed experts,
// then the shared expert).  The router also writes dense_row [T k + T], the
// dense row of every row-space row.  decode_down then runs the down GEMM over
// the row space only, its A rows gathered as act_dense[dense_row[r]], and
// copies those rows to act (the row-space activations) as it stages them.
// Every row's values are bit-identical to the routed path's.
bool decode_dense_applies(size_t T, size_t d, size_t f, size_t E, size_t k, size_t n_shared,
                          int dtype, const void *x, const float *w_router);
int decode_gate_up_router(const void *x, size_t T, size_t d, size_t f, size_t E, size_t k,
                          const float *w_router, const float *w_lds, const float *router_bias,
                          const float *concept_bias, size_t n_concept, float *logits,
                          int32_t *topk_idx, float *topk_w, int32_t *block_counts,
                          int32_t *offsets, int32_t *row_token, float *row_weight,
                          int32_t *token_row, int32_t *dense_row, const void *w_gate_up,
                          void *act_dense, void *stream);
int decode_down(const void *act_dense, const int32_t *dense_row, const int32_t *offsets, size_t T,
                size_t d, size_t f, size_t E, size_t k, const void *w_down, void *y, void *act,
                void *stream);

// Plain grouped GEMM over the engine's row space (no SwiGLU):
// C[r][n] = sum_k A[a_rows ? a_rows[r] : r][k] * B_g[n][k] for the rows r of
// each group g, B_g the g-th packed [Np, K] weight (prichs_pack_weight layout,
// b_group_stride elements apart); columns n < n_store are written.
int grouped_gemm_rows(const void *A, const int32_t *a_rows, size_t lda, const void *B,
                      size_t b_group_stride, size_t Np, size_t K, void *C, size_t ldc,
                      size_t n_store, const int32_t *offsets, size_t G, size_t max_rows,
                      size_t max_group_rows, int dtype, void *stream);

// MoE backward stages (backward.hip); the engine sequences them.
int bwd_rows(const void *x, const void *d_out, const void *y, const int32_t *token_row,
             const float *row_weight, size_t T, size_t k, bool shared, size_t d, int dtype,
             void *dy, void *xg, float *scal, hipStream_t s);
// dA = dY Wd^T (the down weights transposed, packed [G][np_f][d]) with the
// SwiGLU backward in its epilogue: gu [rows][np] (the gate/up pre-activations,
// packed) receives dG, dU in place and dA is never stored.  *fused = false
// (nothing launched) where the tiled bf16 kernel does not apply (f32,
// decode-sized groups, unaligned gu; dact_swiglu_bwd_fusable): the caller
// then runs grouped_gemm_rows into a dA buffer and bwd_swiglu.  a2 (may be
// null): group a2_g's rows a2_row0.. of dY are rows 0.. of a2 (same pitch).
bool dact_swiglu_bwd_fusable(size_t d, size_t np_f, const void *gu, size_t np, size_t f,
                             size_t max_rows, size_t max_group_rows, int dtype);
int grouped_dact_swiglu_bwd(const void *dy, size_t d, const void *w_down_t, size_t b_group_stride,
                            size_t np_f, void *gu, size_t np, size_t f, const int32_t *offsets,
                            size_t G, size_t max_rows, size_t max_group_rows, int dtype,
                            void *stream, bool *fused, const void *a2 = nullptr, size_t a2_g = 0,
                            size_t a2_row0 = 0);
int bwd_swiglu(void *gu, const void *da, size_t rows, size_t f, size_t np, int dtype,
               hipStream_t s);
// part: bf16 split-K partials, bwd_wgrad_part_elems(rows, P, Q) floats.
size_t bwd_wgrad_part_elems(size_t max_rows, size_t P, size_t Q);
// Group g's rows row0 .. row0 + rows - 1 of the row space read from A / B
// (bf16, same row pitch) instead, where those are set: the shared expert's
// rows are x and d_out themselves, which the rows pass then need not copy.
struct WgradAlt {
  const void *A = nullptr, *B = nullptr;
  size_t g = 0, row0 = 0, rows = 0;
};
int bwd_wgrad(bool gateup, const void *A, size_t lda, const void *B, size_t ldb, size_t total_rows,
              const int32_t *offsets, size_t G, size_t E, size_t P, size_t Q, float *out0,
              float *out1, size_t ldo, size_t slot_stride, size_t f, int dtype, float *part,
              int beta, hipStream_t s, const WgradAlt &alt = WgradAlt());
int bwd_combine(const void *dX, const float *scal, const int32_t *topk_idx, const float *topk_w,
                const int32_t *token_row, const float *wrt, size_t T, size_t d, size_t k,
                int weighting, int dtype, float *dlr, void *d_x, int dx_dtype, hipStream_t s);
int bwd_zero_grads(float *d_router, size_t n_router, float *d_gate, float *d_up, float *d_down,
                   size_t slot_stride, size_t G, size_t n_mat, hipStream_t s);
size_t bwd_router_part_elems(size_t max_tokens, size_t k, size_t d, size_t E);
int bwd_router_wgrad(const void *xg, const float *dlr, const int32_t *offsets, size_t T, size_t k,
                     size_t d, size_t E, int dtype, float *part, float *dw, int beta,
                     hipStream_t s);

// Checkpoint reading shared by the engines' upload-from-checkpoint entry
// points: parameter `index` must hold exactly `want` floats (`what` and
// `layer` name it in the error message).
int checkpoint_read_vec(const prichs_checkpoint *ck, size_t index, size_t want,
                        std::vector<float> &out, const char *what, size_t layer);
// One MoE layer's weights in the reference layouts, shared expert first,
// with the pointer arrays prichs_moe_engine_upload takes.
struct CheckpointMoe {
  std::vector<float> router;
  std::vector<std::vector<float>> gate, up, down;
  std::vector<const float *> pg, pu, pd;
};
int checkpoint_moe_weights(const prichs_checkpoint *ck, size_t layer, size_t d, size_t f,
                           size_t E, CheckpointMoe &w);

// prichs_attention_forward, with q rotated by RoPE as the kernel loads it
// when rope_cos is set (the cos / sin tables of prichs_rope_cache, cache_rows
// positions of head_dim / 2 pairs; positions pos_offset .. pos_offset +
// seq_len - 1): the attention of the q that prichs_rope_forward would leave.
int attention_forward_impl(const void *q, size_t ldq, const void *k, size_t ldk, const void *v,
                           size_t ldv, void *o, size_t ldo, size_t batch, size_t seq_len,
                           size_t n_heads, size_t n_kv_heads, size_t head_dim, int dtype,
                           const float *rope_cos, const float *rope_sin, size_t cache_rows,
                           size_t pos_offset, void *stream);

// prichs_router_topk then prichs_permute; when one router workgroup covers
// the batch (decode-sized T) the router writes the permutation itself
// (router.hip).  Same outputs either way.  w_lds (may be null): the router
// weights in the router's LDS layout, W^T [E][d + 4] f32 with zero padding
// (router_lds_layout), which spares each router workgroup the transpose.
int router_topk_permute(const void *x, int x_dtype, const float *w_router,
                        const float *router_bias, const float *concept_bias, size_t n_concept,
                        size_t T, size_t d, size_t E, size_t k, float *logits, int32_t *topk_idx,
                        float *topk_w, int32_t *block_counts, int32_t *offsets,
                        int32_t *row_token, float *row_weight, int32_t *token_row, void *stream,
                        const float *w_lds = nullptr);
// prichs_router_topk with the W^T copy above (may be null).
int router_topk_lds(const void *x, int x_dtype, const float *w_router, const float *w_lds,
                    const float *router_bias, const float *concept_bias, size_t n_concept,
                    size_t T, size_t d, size_t E, size_t k, float *logits, int32_t *topk_idx,
                    float *topk_w, int32_t *block_counts, void *stream);
// Elements of that copy (0 when the router kernel that reads it does not
// apply to the shape), and the copy of host weights W [d][E] into host memory.
size_t router_lds_layout_elems(size_t d, size_t E);
void router_lds_layout(const float *w_router, size_t d, size_t E, float *out);

// prichs_moe_combine; y_last_use: no later kernel reads y, so its loads are
// non-temporal (the same results; elementwise.hip).
int moe_combine(const void *y, int y_dtype, const int32_t *topk_idx, const float *topk_w,
                const int32_t *token_row, size_t T, size_t d, size_t k, int has_shared, void *out,
                int out_dtype, void *stream, bool y_last_use);
// moe_out = the MoE combine (bf16) and out = res + moe_out (the block's final
// residual add) in one kernel (elementwise.hip); y_last_use as above.
int moe_combine_residual(const void *y, const int32_t *topk_idx, const float *topk_w,
                         const int32_t *token_row, size_t T, size_t d, size_t k, int has_shared,
                         void *moe_out, const float *res, void *out, int out_dtype, void *stream,
                         bool y_last_use = false);
// prichs_moe_engine_forward whose combine also adds the f32 residual:
// moe_out gets the layer output (bf16), out = residual + moe_out (engine.hip).
int moe_engine_forward_residual(prichs_moe_engine *eng, const void *x, size_t T,
                                const float *concept_bias, size_t n_concept, void *moe_out,
                                const float *residual, void *out, int out_dtype, void *stream);

// The block's residual add and post-attention norm in one pass:
// x1 = a + b (f32), out = rms_norm(x1, w) (bf16) (elementwise.hip).
int add_rmsnorm_forward(const void *a, int a_dtype, const void *b, int b_dtype, float *x1,
                        const float *w, void *out, size_t T, size_t d, float eps, void *stream);

}  // namespace prichs
