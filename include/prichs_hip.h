/*
 * prichs_hip.h -- C ABI of libprichs_hip.so, the MI355X (gfx950) MoE
 * feed-forward hot path of PRICHS.
 *
 * Reference paths below are relative to the PRICHS source tree.
 *
 * Four groups of entry points:
 *
 *  1. Legacy launchers with the exact signatures of the reference's CUDA
 *     launchers (crates/prichs-cuda/src/kernels.cu; Rust extern block at
 *     crates/prichs-cuda/src/engine.rs:89-272), so the existing Rust extern
 *     declarations link against this library unchanged.  Like the originals
 *     they return void; failures are recorded in prichs_last_error().
 *
 *  2. Stage entry points of the device-resident MoE forward (router + top-k,
 *     permutation, grouped expert GEMMs, combine) and the memory-bound
 *     RMSNorm / RoPE kernels.  They replace the host-side routing and the
 *     per-expert cuBLAS loop of crates/prichs-model/src/model.rs:1125-1177.
 *
 *  3. An engine handle that owns packed weights and workspace and runs the
 *     whole MoELayer forward (crates/prichs-model/src/moe.rs:93-225) on one
 *     stream with no host round trip and no allocation per call (and a
 *     PrichsBlock engine around it); the same engine runs the layer's
 *     training-step backward (crates/prichs-cuda/src/engine.rs:2242-2789).
 *
 *  4. A reader of the reference's checkpoint files that uploads a block's
 *     weights into those engines.
 *
 * Conventions:
 *  - Every non-legacy entry point returns PRICHS_OK (0) or a negative status.
 *    The message of the last failure on the calling thread is available from
 *    prichs_last_error().  Argument checks run before any HIP call, so invalid
 *    arguments are reported even on a machine without a GPU.
 *  - Pointers named dev_* or documented as device memory are device pointers.
 *    `stream` is a hipStream_t (NULL = the default stream).  Calls are
 *    asynchronous on that stream unless stated otherwise.
 *  - Weights are accepted in the reference layouts: f32 row-major [K, N]
 *    ("x @ W" form): gate/up [d, f], down [f, d], router [d, E]
 *    (crates/prichs-model/src/moe.rs:16-18, 74).
 *  - dtype codes: PRICHS_DTYPE_F32 (IEEE binary32) and PRICHS_DTYPE_BF16
 *    (bfloat16 bit patterns in uint16 storage).
 *  - Results of every entry point are deterministic: no floating-point
 *    atomics on any path except the legacy launch_moe_scatter_add and
 *    launch_moe_scatter_add_grad, which keep the reference's atomicAdd
 *    semantics.
 */
#ifndef PRICHS_HIP_H
#define PRICHS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------- */
/* Status codes, dtypes, diagnostics                                       */
/* ---------------------------------------------------------------------- */
enum {
  PRICHS_OK = 0,
  PRICHS_ERR_INVALID_ARGUMENT = -1, /* null pointer, bad shape, bad E/k   */
  PRICHS_ERR_CAPACITY = -2,         /* exceeds a preallocated capacity    */
  PRICHS_ERR_HIP = -3,              /* a HIP runtime call failed          */
  PRICHS_ERR_UNSUPPORTED = -4,      /* valid but unsupported shape/dtype  */
  PRICHS_ERR_STATE = -5             /* e.g. forward before weights upload */
};

enum { PRICHS_DTYPE_F32 = 0, PRICHS_DTYPE_BF16 = 1 };

/* Limits of the stage kernels. */
#define PRICHS_MAX_EXPERTS 64 /* routed experts E                       */
#define PRICHS_MAX_TOPK 8     /* k                                      */

/* Message of the last failure on the calling thread ("" if none). */
const char *prichs_last_error(void);
/* Clears the calling thread's last error. */
void prichs_clear_error(void);
/* ABI version of this header (major * 10000 + minor * 100 + patch). */
int prichs_abi_version(void);
/* The current device's compute units, peak engine and memory clocks (kHz)
 * and memory bus width (bits), for rooflines (any output may be NULL). */
int prichs_device_caps(int *cus, int *clock_khz, int *mem_clock_khz,
                       int *mem_bus_bits);

/* ---------------------------------------------------------------------- */
/* 1. Legacy launchers (identical signatures to the reference)             */
/* ---------------------------------------------------------------------- */

/* Replaces launch_rmsnorm_forward (crates/prichs-cuda/src/kernels.cu:403-419,
 * kernel 329-362).  Per row: rstd = 1/sqrt(mean(x^2) + eps),
 * out = (x * rstd) * w; writes rstd[t].  f32 [seq_len, hidden_dim]. */
void launch_rmsnorm_forward(const float *dev_x, const float *dev_weight,
                            float *dev_out, float *dev_rstd_out, size_t seq_len,
                            size_t hidden_dim, float eps, void *stream);

/* Replaces launch_swiglu_forward (kernels.cu:482-496, kernel 444-457).
 * out = silu(g) * u with silu(g) = g / (1 + exp(-g)) (the CPU formula of
 * crates/prichs-core/src/ops.rs:137-140). */
void launch_swiglu_forward(const float *dev_gate, const float *dev_up,
                           float *dev_out, size_t total_elements, void *stream);

/* Replaces launch_rope (kernels.cu:554-572, kernel 520-552).  In-place
 * rotation of interleaved pairs of [seq_len, num_heads, head_dim] by
 * cos/sin[t * head_dim/2 + i]; sin is multiplied by (float)backward_sign,
 * whatever its value (+1 forward, -1 inverse), as in the original.  Like the
 * original it has no position offset; prichs_rope_forward has one. */
void launch_rope(float *dev_q_or_k, const float *dev_cos_cache,
                 const float *dev_sin_cache, size_t seq_len, size_t num_heads,
                 size_t head_dim, int backward_sign, void *stream);

/* Replaces launch_moe_gather (kernels.cu:993-1007, kernel 888-904).
 * out[i, :] = in[token_indices[i], :]. */
void launch_moe_gather(const float *dev_in, const int *dev_token_indices,
                       float *dev_out, size_t n_tokens, size_t hidden_dim,
                       void *stream);

/* Replaces launch_moe_scatter_add (kernels.cu:1009-1024, kernel 906-924).
 * accum[token_indices[i], :] += weights[i] * exp_out[i, :] (atomic add, as in
 * the reference; with distinct indices -- the reference's only use -- the
 * result is deterministic). */
void launch_moe_scatter_add(const float *dev_exp_out,
                            const int *dev_token_indices,
                            const float *dev_weights, float *dev_accum_out,
                            size_t n_tokens, size_t hidden_dim, void *stream);

/* The backward launchers (Rust extern block engine.rs:152-160, 244-271).
 * Replaces launch_swiglu_backward (kernels.cu:498-514, kernel 459-480):
 * sig = 1/(1+exp(-g)), dup = dact*g*sig, dgate = (dact*up)*sig*(1+g*(1-sig)). */
void launch_swiglu_backward(const float *dev_dact, const float *dev_gate,
                            const float *dev_up, float *dev_dgate, float *dev_dup,
                            size_t total_elements, void *stream);

/* Replaces launch_moe_backward_gather_weighted (kernels.cu:1026-1041, kernel
 * 926-944): d_y_e[i, :] = weights[i] * d_moe[token_indices[i], :]. */
void launch_moe_backward_gather_weighted(const float *dev_d_moe,
                                         const int *dev_token_indices,
                                         const float *dev_weights, float *dev_d_y_e,
                                         size_t n_tokens, size_t hidden_dim,
                                         void *stream);

/* Replaces launch_moe_router_dot (kernels.cu:1043-1057, kernel 946-969):
 * scalars_out[i] = sum_c exp_out[i, c] * d_moe[token_indices[i], c] (one wave
 * per row, summed in a fixed order). */
void launch_moe_router_dot(const float *dev_exp_out, const float *dev_d_moe,
                           const int *dev_token_indices, float *dev_scalars_out,
                           size_t n_tokens, size_t hidden_dim, void *stream);

/* Replaces launch_moe_scatter_add_grad (kernels.cu:1059-1075, kernel 971-991):
 * d_normed2[token_indices[i], :] += weights[i] * (d_x_e[i, :] + d_x_e_tmp[i, :])
 * (atomic add, as in the reference; order-free for the distinct indices of one
 * expert's token list). */
void launch_moe_scatter_add_grad(const float *dev_d_x_e, const float *dev_d_x_e_tmp,
                                 const int *dev_token_indices,
                                 const float *dev_weights, float *dev_d_normed2,
                                 size_t n_tokens, size_t hidden_dim, void *stream);

/* ---------------------------------------------------------------------- */
/* 2. Stage entry points                                                   */
/* ---------------------------------------------------------------------- */

/* Number of token blocks the router uses for T tokens and E experts; the
 * block_counts workspace of prichs_router_topk holds blocks * E int32. */
size_t prichs_router_num_blocks(size_t T, size_t E);

/* Router + top-k gating.  Replaces forward_gemm(router) + the host loop
 * (crates/prichs-cuda/src/engine.rs:757-826; crates/prichs-model/src/
 * model.rs:1136-1151) and restates moe.rs:113-142 / ops.rs:219-248 on device:
 *   raw[t,e] = sum_k x[t,k] * W[k,e]   (k ascending, no FMA: bit-exact with
 *                                        the reference CPU GEMM),
 *   adj = (raw + router_bias[e]) (+ concept_bias[e] for e < n_concept),
 *   top-k by a stable descending order of adj (ties -> lower expert index),
 *   weights = softmax of the RAW logits of the selected experts,
 *   w = e_i / (sum e + 1e-9).
 * x: [T, d] of x_dtype (device).  w_router: f32 [d, E] (device).
 * router_bias: f32 [E] (device).  concept_bias: f32 [n_concept] (device, may
 * be NULL).  Outputs (device): logits f32 [T, E] (may be NULL), topk_idx int32
 * [T, k], topk_w f32 [T, k], block_counts int32 [prichs_router_num_blocks*E]
 * (per-block expert histogram consumed by prichs_permute).
 * Limits: 1 <= E <= PRICHS_MAX_EXPERTS, 1 <= k <= min(E, PRICHS_MAX_TOPK). */
int prichs_router_topk(const void *x, int x_dtype, const float *w_router,
                       const float *router_bias, const float *concept_bias,
                       size_t n_concept, size_t T, size_t d, size_t E, size_t k,
                       float *logits, int32_t *topk_idx, float *topk_w,
                       int32_t *block_counts, void *stream);

/* Token permutation (stable counting sort by expert id).  Restates the
 * binning of crates/prichs-model/src/moe.rs:121, 137-141, 149-164: rows are
 * ordered by (expert ascending, token ascending).  Outputs (device):
 *   offsets   int32 [E + 2]: rows of routed expert e are
 *             [offsets[e], offsets[e+1]); offsets[E] = T*k; the shared
 *             expert's rows are [T*k, offsets[E+1] = T*k + T).
 *   row_token int32 [T*k + T]: token of each row (shared rows: t -> t).
 *   row_weight f32 [T*k]: gate weight of each routed row.
 *   token_row int32 [T*k]: row of (token t, slot s) at t*k + s.
 * block_counts comes from prichs_router_topk with the same T, E. */
int prichs_permute(const int32_t *topk_idx, const float *topk_w,
                   const int32_t *block_counts, size_t T, size_t E, size_t k,
                   int32_t *offsets, int32_t *row_token, float *row_weight,
                   int32_t *token_row, void *stream);

/* Packed expert-weight layouts used by the grouped GEMMs (host functions,
 * no GPU needed).  il = prichs_gate_up_interleave(dtype) is the gate/up
 * interleave of the kernel that consumes the buffer.
 *
 * gate/up, one expert: packed [Np, K = d] with K contiguous, Np =
 *   roundup(2 * roundup(f, il), N tile) (N tile 256 for bf16, 128 for f32);
 *   packed row p = 2*il*b + q holds column il*b + q of gate (q < il) or
 *   column il*b + q - il of up (q >= il), zero when that column is >= f.
 * down, one expert: packed [roundup(d, 256), K = f] = W_down^T, zero rows
 *   past d.
 * Element type: dtype (bf16 by round-to-nearest-even from f32).
 * Storage order of a packed [Np, K]: f32 row-major (element (n, k) at
 *   n*K + k); bf16 fragment-major, the operand layout of the MFMA
 *   v_mfma_f32_16x16x32_bf16: element (n, k) at
 *   ((n/16 * K/32 + k/32) * 64 + n%16 + 16*((k%32)/8)) * 8 + k%8,
 *   so each 16-row x 32-k fragment is one contiguous KiB. */
size_t prichs_gate_up_interleave(int dtype);
size_t prichs_packed_gate_up_elems(size_t d, size_t f, int dtype);
size_t prichs_packed_down_elems(size_t d, size_t f, int dtype);
int prichs_pack_gate_up(const float *gate, const float *up, size_t d, size_t f,
                        int dtype, void *packed_out);
int prichs_pack_down(const float *down, size_t d, size_t f, int dtype,
                     void *packed_out);

/* Grouped gate/up GEMM with the SwiGLU epilogue fused.  Replaces the gate and
 * up SGEMMs plus launch_swiglu_forward of gpu_moe_forward_shared /
 * gpu_moe_forward_expert (crates/prichs-cuda/src/engine.rs:1957-1999,
 * 2112-2153); math of crates/prichs-model/src/moe.rs:166-169 and 103-105.
 * For every row r of group g (rows [offsets[g], offsets[g+1])):
 *   act[r, :] = silu(x[row_token[r]] @ Wg_g) * (x[row_token[r]] @ Wu_g).
 * Groups 0..G-1 use packed weights w_packed + g * prichs_packed_gate_up_elems.
 * With the offsets/row_token of prichs_permute, G = E + 1 covers the routed
 * experts (g < E) and the shared expert (g = E, its weights packed last).
 * x [T, d], act [offsets[G], f] and the weights share `dtype`; fp32
 * accumulation.  Requires d % 64 == 0 and f % 64 == 0 for bf16, d % 16 == 0
 * and f % 16 == 0 for f32.  max_rows bounds offsets[G] (sizes the launch);
 * bf16 launches with max_rows <= 64 stream the weights through a skinny
 * (decode) kernel instead of the 256x256-tiled one. */
int prichs_grouped_gate_up_swiglu(const void *x, const int32_t *row_token,
                                  const int32_t *offsets, size_t G,
                                  size_t max_rows, const void *w_packed,
                                  size_t d, size_t f, int dtype, void *act,
                                  void *stream);

/* Grouped down GEMM: y[r, :] = act[r, :] @ Wd_g for the rows of each group.
 * Replaces the down SGEMMs (engine.rs:2002-2017, 2156-2171; moe.rs:170,106).
 * act [offsets[G], f], y [offsets[G], d] of `dtype`; fp32 accumulation. */
int prichs_grouped_down(const void *act, const int32_t *offsets, size_t G,
                        size_t max_rows, const void *w_packed, size_t d,
                        size_t f, int dtype, void *y, void *stream);

/* Deterministic combine.  Replaces launch_moe_scatter_add + the shared
 * initialisation (kernels.cu:906-924; engine.rs:2002-2017, 2226-2239) and
 * restates moe.rs:146, 177-184: per token,
 *   out = shared_y[t]; then for its experts in ASCENDING expert id:
 *   out = out + w * y[row]   (product rounded, then sum).
 * y [T*k + T*has_shared, d] of y_dtype laid out as by prichs_permute (shared
 * rows last), out [T, d] of out_dtype. */
int prichs_moe_combine(const void *y, int y_dtype, const int32_t *topk_idx,
                       const float *topk_w, const int32_t *token_row,
                       size_t T, size_t d, size_t k, int has_shared, void *out,
                       int out_dtype, void *stream);

/* RMSNorm (memory-bound).  crates/prichs-core/src/ops.rs:109-135:
 * out = (x * inv) * w, inv = 1/sqrt(sum(x^2)/d + eps); rstd[t] = inv
 * (rstd may be NULL).  x/out dtypes independent; w is f32 [d]. */
int prichs_rmsnorm_forward(const void *x, int x_dtype, const float *w,
                           void *out, int out_dtype, float *rstd, size_t T,
                           size_t d, float eps, void *stream);

/* RoPE (memory-bound, in place).  crates/prichs-core/src/backward.rs:160-188
 * for `batch` independent sequences: qk [batch, seq_len, n_heads, head_dim],
 * position of row s = s + pos_offset, cache f32 [*, head_dim/2] from the
 * host (backward.rs:136-157); sign = +1 forward, -1 inverse rotation.
 * cache_rows bounds the positions (seq_len + pos_offset <= cache_rows). */
int prichs_rope_forward(void *qk, int dtype, const float *cos_cache,
                        const float *sin_cache, size_t cache_rows, size_t batch,
                        size_t seq_len, size_t n_heads, size_t head_dim,
                        size_t pos_offset, int sign, void *stream);

/* RoPE with a row stride (elements between consecutive rows of qk), for Q
 * or K living inside a fused [rows, q | k | v] projection buffer.  Same
 * arithmetic as prichs_rope_forward (backward.rs:160-188). */
int prichs_rope_forward_ld(void *qk, size_t row_stride, int dtype,
                           const float *cos_cache, const float *sin_cache,
                           size_t cache_rows, size_t batch, size_t seq_len,
                           size_t n_heads, size_t head_dim, size_t pos_offset,
                           int sign, void *stream);

/* out = a + b element-wise in f32 arithmetic; each operand bf16 or f32.
 * Replaces add_tensors (crates/prichs-core/src/ops.rs:250-267) for the
 * block's residual connections.  n % 8 == 0, 16-byte aligned operands. */
int prichs_add(const void *a, int a_dtype, const void *b, int b_dtype,
               void *out, int out_dtype, size_t n, void *stream);

/* dst = src, bytes a multiple of 16, both 16-byte aligned, no overlap: a
 * streaming copy kernel of this library (16 bytes per lane, 8 chunks per
 * thread in flight), the practical HBM yardstick that the memory-bound
 * stages are measured against.  No counterpart in the reference. */
int prichs_hbm_copy(const void *src, void *dst, size_t bytes, void *stream);

/* Dense GEMM C[M, N] = A[M, K] @ W on the bf16 (or f32) MFMA kernel of the
 * grouped GEMMs: replaces matmul_2d's device dispatch / forward_gemm
 * (crates/prichs-core/src/ops.rs:24-31; crates/prichs-cuda/src/engine.rs:
 * 757-826) for the block's projections.  W comes from prichs_pack_weight
 * (the packed-down storage order above: [roundup(N, 256), K] = W^T).
 * Row strides lda (multiple of 8) and ldc (multiple of 4); K and N multiples
 * of 64 (bf16) or 16 (f32); fp32 accumulation. */
size_t prichs_packed_weight_elems(size_t K, size_t N, int dtype);
int prichs_pack_weight(const float *w, size_t K, size_t N, int dtype,
                       void *packed_out);
int prichs_gemm(const void *a, size_t lda, size_t M, size_t K,
                const void *w_packed, size_t N, void *c, size_t ldc, int dtype,
                void *stream);

/* Causal GQA self-attention forward (flash-style; bf16 in/out, fp32
 * softmax and accumulation).  Restates the per-head attention of
 * crates/prichs-model/src/attention.rs:94-149 -- query head h attends with
 * kv head h / (n_heads / n_kv_heads), scores (q . k) / sqrt(head_dim) over
 * j <= i, softmax over the causal row -- for `batch` independent sequences:
 * row r of sequence b is row b * seq_len + r of q/k/v/o; head h of q and o
 * starts at column h * head_dim, kv head j of k and v at column j * head_dim
 * (leading dimensions ldq/ldk/ldv/ldo, multiples of 8).  Replaces the
 * materialised-score attention of gpu_batched_attention_forward
 * (crates/prichs-cuda/src/engine.rs:1181-1405).  head_dim must be 128. */
int prichs_attention_forward(const void *q, size_t ldq, const void *k,
                             size_t ldk, const void *v, size_t ldv, void *o,
                             size_t ldo, size_t batch, size_t seq_len,
                             size_t n_heads, size_t n_kv_heads,
                             size_t head_dim, int dtype, void *stream);

/* The same attention with RoPE applied to q as the kernel loads it: query
 * row r of sequence b is rotated at position pos_offset + r with the tables
 * cos / sin [cache_rows, head_dim / 2] of prichs_rope_cache (device memory),
 * by the interleaved-pair rotation of crates/prichs-core/src/backward.rs:
 * 160-188 with the same roundings as prichs_rope_forward, so the output is
 * bit-identical to prichs_rope_forward on q followed by
 * prichs_attention_forward.  k must be rotated already (the reference's
 * SelfAttention::forward_with_rope rotates q and k, attention.rs:56-92).
 * seq_len + pos_offset <= cache_rows.  The block engine runs its attention
 * this way (q is never written back rotated). */
int prichs_attention_forward_rope_q(const void *q, size_t ldq, const void *k,
                                    size_t ldk, const void *v, size_t ldv, void *o,
                                    size_t ldo, size_t batch, size_t seq_len,
                                    size_t n_heads, size_t n_kv_heads,
                                    size_t head_dim, int dtype, const float *rope_cos,
                                    const float *rope_sin, size_t cache_rows,
                                    size_t pos_offset, void *stream);

/* f32 causal attention of one sequence with the probabilities kept: the
 * per-head computation of crates/prichs-model/src/attention.rs:96-149 (scores
 * (q . k) / sqrt(head_dim), sequential dot products; row max, expf, sum,
 * times 1 / max(sum, 1e-9); context sum over keys ascending) for the
 * reference's host-slice gpu_batched_attention_forward
 * (crates/prichs-cuda/src/engine.rs:1181-1405), which returns these
 * probabilities.  q [T, n_heads * head_dim], k / v [T, n_kv_heads * head_dim]
 * (query head h reads kv head h / (n_heads / n_kv_heads)); probs
 * [n_heads, T, T] (zeros past the diagonal) and ctx [T, n_heads * head_dim]
 * (the heads concatenated); all f32 device memory, contiguous.  seq_len <=
 * 16384 (PRICHS_ERR_UNSUPPORTED beyond). */
int prichs_attention_probs_f32(const float *q, const float *k, const float *v,
                               float *probs, float *ctx, size_t seq_len,
                               size_t n_heads, size_t n_kv_heads, size_t head_dim,
                               void *stream);

/* RoPE cos/sin tables on the host (no GPU needed): replaces
 * precompute_rope_cache (crates/prichs-core/src/backward.rs:136-157).
 * cos/sin [max_seq_len, head_dim/2]: freq_i = 1/theta^(2i/hd) (libm powf),
 * angle = (float)t * freq_i, libm cosf/sinf -- bit-identical to the
 * reference's f32 computation on the same libm.  Upload the tables for
 * prichs_rope_forward / launch_rope. */
int prichs_rope_cache(size_t max_seq_len, size_t head_dim, float theta,
                      float *cos_out, float *sin_out);

/* ---------------------------------------------------------------------- */
/* 3. MoE engine (owns packed weights + workspace; replaces the MoE part of */
/*    GpuModelEngine: engine.rs:363-649, 668-689, 1917-2239)               */
/* ---------------------------------------------------------------------- */
typedef struct prichs_moe_engine prichs_moe_engine;

/* Creates an engine for one MoE layer on the current HIP device.
 * n_shared is 0 or 1 (the reference has 1, moe.rs:61).  dtype is the
 * arithmetic type of the expert GEMMs and activations (F32 or BF16).
 * max_tokens is the largest T a forward may use; all workspace is
 * allocated here (forward allocates nothing). */
int prichs_moe_engine_create(size_t d, size_t f, size_t E, size_t k,
                             size_t n_shared, int dtype, size_t max_tokens,
                             prichs_moe_engine **out);
int prichs_moe_engine_destroy(prichs_moe_engine *eng);

/* Uploads weights given in the reference layouts (host f32): router [d, E],
 * router_bias [E] (may be NULL = zeros, moe.rs:75), and arrays of
 * n_shared + E pointers (shared expert first, then routed 0..E-1) to
 * gate [d, f], up [d, f], down [f, d].  Synchronous.  Replaces
 * upload_weights (engine.rs:668-689) for one layer; packs to the kernels'
 * layouts. */
int prichs_moe_engine_upload(prichs_moe_engine *eng, const float *w_router,
                             const float *router_bias,
                             const float *const *gate, const float *const *up,
                             const float *const *down);

/* Replaces the host-side aux-free bias (moe.rs:60, 228-245): host f32 [E]. */
int prichs_moe_engine_set_router_bias(prichs_moe_engine *eng,
                                      const float *router_bias);

/* The aux-loss-free bias update on device: MoELayer::update_aux_free_bias
 * (crates/prichs-model/src/moe.rs:228-245) as its call site drives it
 * (crates/prichs-model/src/model.rs:1541-1547): counts = assignments per
 * expert in the last forward (the permutation's group sizes), total_tokens =
 * that forward's T; bias[i] += gamma * (k/E - counts[i]/T) in f32.  Enqueued
 * on `stream` after the forward; no-op after a forward of T = 0. */
int prichs_moe_engine_update_router_bias(prichs_moe_engine *eng, float gamma,
                                         void *stream);
/* Copies the current router bias f32 [E] to host memory (synchronous). */
int prichs_moe_engine_get_router_bias(const prichs_moe_engine *eng, float *out);

/* Full MoELayer forward (moe.rs:93-225) on device: x [T, d] of the engine's
 * dtype (device), optional concept bias f32 [n_concept] (device, may be
 * NULL), out [T, d] of out_dtype (device).  T <= max_tokens. */
int prichs_moe_engine_forward(prichs_moe_engine *eng, const void *x, size_t T,
                              const float *concept_bias, size_t n_concept,
                              void *out, int out_dtype, void *stream);

/* Device views of the last forward's intermediates (the reference's MoEStash,
 * moe.rs:32-53): router logits f32 [T, E], selected experts int32 [T, k],
 * gate weights f32 [T, k], offsets int32 [E + 2], row_token int32 [T*k + T],
 * row_weight f32 [T*k], token_row int32 [T*k], act [T*k + T, f] and
 * y [T*k + T, d] of the engine dtype (routed rows in permuted order, shared
 * rows last).  Valid until the next forward. */
typedef struct prichs_moe_stash {
  size_t T;
  const float *router_logits;
  const int32_t *selected_experts;
  const float *gating_weights;
  const int32_t *offsets;
  const int32_t *row_token;
  const float *row_weight;
  const int32_t *token_row;
  const void *act;
  const void *y;
} prichs_moe_stash;
int prichs_moe_engine_stash(const prichs_moe_engine *eng,
                            prichs_moe_stash *out);

/* Stage timing.  set_timing(eng, n) creates events for n forwards (0 turns
 * timing off); each following forward, up to n of them, records HIP events
 * on its stream between its stages, with no host synchronisation.
 * stage_ms waits for those forwards and writes the AVERAGE milliseconds of:
 * [0] router, [1] permute, [2] gate/up GEMM, [3] down GEMM, [4] combine,
 * [5] whole forward; *n_forwards (may be NULL) gets the number averaged.
 * It then re-arms recording for another n forwards.  When one router
 * workgroup covers the batch (decode-sized T, bf16, one shared expert, 5-8
 * routed experts, d % 128 == 0, no backward enabled), the router and the
 * permutation run inside the gate/up launch, which covers every token of
 * every expert, and the down GEMM gathers the routed rows: [0] and [1] then
 * time only event gaps and [2] covers the router too.  The stash's rows and
 * every output are bit-identical either way.  Each event
 * costs a few microseconds on the stream, so time throughput with timing
 * off. */
#define PRICHS_NUM_STAGES 6
int prichs_moe_engine_set_timing(prichs_moe_engine *eng, int max_forwards);
int prichs_moe_engine_stage_ms(prichs_moe_engine *eng, float *ms_out,
                               int *n_forwards);

/* ---- Backward: the training step's MoE gradients ------------------------
 * Replaces GpuModelEngine::gpu_moe_init_backward, gpu_moe_backward_expert
 * (per routed expert), gpu_moe_backward_shared and gpu_moe_backward_router
 * (crates/prichs-cuda/src/engine.rs:2242-2789) as Model::train_step drives
 * them (crates/prichs-model/src/model.rs:1474-1561), with the router VJP
 * moe_router_unbiased_backward (crates/prichs-core/src/backward.rs:269-287)
 * on device.  One call covers every expert; nothing is summed with atomics,
 * so the result is deterministic. */

/* Allocates the backward's workspace (about (T*(k+1)) * (2f + 2d) elements
 * of the engine dtype for max_tokens T) and makes the next uploads also pack
 * the transposed weights the input-gradient products need; from then on each
 * forward's gate/up GEMM also stores its pre-activations for the backward.
 * Call after create and before upload / upload_checkpoint.  Needs
 * n_shared = 1 (the reference's layer, moe.rs:61).  Synchronous. */
int prichs_moe_engine_enable_backward(prichs_moe_engine *eng);

/* Caller-owned f32 gradient buffers (device) in the reference's layouts:
 * d_router [d, E]; per expert slot s (0 = shared expert, 1 + e = routed
 * expert e) d_gate + s*slot_stride and d_up + s*slot_stride [d, f],
 * d_down + s*slot_stride [f, d].  With the reference's parameter order
 * (model.rs:312-338) d_up = d_gate + d*f, d_down = d_gate + 2*d*f and
 * slot_stride = 3*d*f.  16-byte aligned.  Every buffer becomes
 * beta * buffer + gradient: beta = 1 adds to it like the reference's dev_grads
 * (cuBLAS beta = 1; gradient accumulation over micro-batches,
 * model.rs:1209-1215); beta = 0 overwrites it, the same as zero_grads
 * (engine.rs:710-720) before the call (model.rs:1198-1207), and needs no read
 * of the old values. */
typedef struct prichs_moe_grads {
  float *d_router;
  float *d_gate;
  float *d_up;
  float *d_down;
  size_t slot_stride;
  int beta;
} prichs_moe_grads;

/* Gradients of the layer output's loss given d_out = dL/d(moe output)
 * [T, d] (engine dtype, device), for the batch of the forward that ran just
 * before on this engine (same x [T, d], device): writes d_x [T, d] (d_x_dtype,
 * device; the reference's d_normed2) and the weight gradients into *grads
 * (beta above).  dx_weighting = 2 reproduces the reference, whose routed input
 * gradient carries the gate weight twice (its gather scales dY by w,
 * kernels.cu:926-944, and its scatter scales dX again, kernels.cu:971-991);
 * dx_weighting = 1 is the chain rule.  The weight gradients do not depend on
 * it.  The forward's stash is consumed (its buffers are reused): one
 * backward per forward.  x, d_out and d_x are 16-byte aligned. */
int prichs_moe_engine_backward(prichs_moe_engine *eng, const void *x,
                               const void *d_out, size_t T, void *d_x,
                               int d_x_dtype, const prichs_moe_grads *grads,
                               int dx_weighting, void *stream);

/* Backward stage timing: with backward enabled, set_timing(eng, n) also
 * records events in each of the next n backwards, and backward_stage_ms
 * writes their AVERAGE milliseconds: [0] gate/up pre-activations (empty:
 * the forward's gate/up GEMM writes them once the backward is enabled), [1] rows
 * pass (dY, gathered x, router scalars), [2] dW_down, [3] dA = dY Wd^T
 * (with the SwiGLU backward in its epilogue for bf16 at tiled sizes), [4]
 * SwiGLU backward (then empty), [5] dX = [dG dU] [Wg Wu]^T, [6] combine (router
 * VJP, d_x), [7] dW_gate / dW_up, [8] dW_router, [9] whole backward. */
#define PRICHS_NUM_BWD_STAGES 10
int prichs_moe_engine_backward_stage_ms(prichs_moe_engine *eng, float *ms_out,
                                        int *n_backwards);

/* ---------------------------------------------------------------------- */
/* 4. PrichsBlock engine (crates/prichs-model/src/block.rs:50-68): RMSNorm,  */
/*    GQA attention with RoPE, residual, RMSNorm, the MoE engine, residual. */
/* ---------------------------------------------------------------------- */
typedef struct prichs_block_engine prichs_block_engine;

/* Creates a block engine (bf16 activations and weights, fp32 accumulation,
 * f32 residual stream) for up to max_tokens rows and positions below
 * max_seq_len; the RoPE tables for rope_theta are built here
 * (prichs_rope_cache).  head_dim = d / n_heads must be 128. */
int prichs_block_engine_create(size_t d, size_t n_heads, size_t n_kv_heads,
                               size_t f, size_t E, size_t k, size_t n_shared,
                               size_t max_tokens, size_t max_seq_len,
                               float rope_theta, float eps,
                               prichs_block_engine **out);
int prichs_block_engine_destroy(prichs_block_engine *eng);

/* Host f32 weights in the reference layouts (block.rs:15-48,
 * attention.rs:17-26): input_norm / post_attn_norm [d], wq [d, d],
 * wk / wv [d, n_kv_heads * head_dim], wo [d, d]; the MoE weights as for
 * prichs_moe_engine_upload.  Synchronous. */
int prichs_block_engine_upload(prichs_block_engine *eng, const float *input_norm,
                               const float *post_attn_norm, const float *wq,
                               const float *wk, const float *wv, const float *wo,
                               const float *w_router, const float *router_bias,
                               const float *const *gate, const float *const *up,
                               const float *const *down);

/* x: bf16 [batch * seq_len, d] (device), `batch` independent sequences at
 * positions pos_offset .. pos_offset + seq_len - 1; out [batch * seq_len, d]
 * of out_dtype (device).  concept_bias as for prichs_moe_engine_forward. */
int prichs_block_engine_forward(prichs_block_engine *eng, const void *x,
                                size_t batch, size_t seq_len, size_t pos_offset,
                                const float *concept_bias, size_t n_concept,
                                void *out, int out_dtype, void *stream);

/* Device views of the last forward's intermediates: normed1 bf16 [T, d],
 * qkv bf16 [T, d + 2 * n_kv_heads * head_dim] (k after RoPE; q as projected:
 * the attention kernel rotates q as it loads it), attn bf16 [T, d]
 * (concatenated heads), attn_out bf16 [T, d] (after Wo),
 * x1 f32 [T, d], normed2 bf16 [T, d], moe_out bf16 [T, d], and the embedded
 * MoE engine (for prichs_moe_engine_stash).  Valid until the next forward. */
typedef struct prichs_block_stash {
  size_t T;
  const void *normed1;
  const void *qkv;
  const void *attn;
  const void *attn_out;
  const float *x1;
  const void *normed2;
  const void *moe_out;
  const prichs_moe_engine *moe;
} prichs_block_stash;
int prichs_block_engine_stash(const prichs_block_engine *eng,
                              prichs_block_stash *out);

/* ---------------------------------------------------------------------- */
/* 5. Checkpoint ingestion: the reference's weight files                    */
/*    (Model::save_checkpoint / load_checkpoint,                            */
/*    crates/prichs-model/src/model.rs:1648-1736)                           */
/* ---------------------------------------------------------------------- */
typedef struct prichs_checkpoint prichs_checkpoint;

/* Opens a weight file and indexes its parameters without reading their
 * payloads.  PRICHS02 (little endian): "PRICHS02", step u64, loss f32,
 * count u64, then count x (len u64, len f32) in the order of
 * Model::get_parameter_tensors (model.rs:312-338).  A legacy "PRICHS_W"
 * file (model.rs:1707-1729: embedding table and final norm only) opens with
 * format 1 and no indexed parameters.  A bad magic, a header or payload
 * running past the end of the file fails with PRICHS_ERR_INVALID_ARGUMENT.
 * Host only (no GPU needed). */
int prichs_checkpoint_open(const char *path, prichs_checkpoint **out);
int prichs_checkpoint_close(prichs_checkpoint *ck);
/* step and loss from the header, the number of indexed parameters and the
 * format (2 = PRICHS02, 1 = PRICHS_W); any output pointer may be NULL. */
int prichs_checkpoint_info(const prichs_checkpoint *ck, uint64_t *step, float *loss,
                           size_t *n_params, int *format);
/* Element count of parameter `index`. */
int prichs_checkpoint_param_len(const prichs_checkpoint *ck, size_t index, size_t *len);
/* Reads parameter `index` (f32, len must equal its element count) into host
 * memory. */
int prichs_checkpoint_read(const prichs_checkpoint *ck, size_t index, float *dst, size_t len);

/* Slots of one block's parameters (model.rs:318-333); routed expert e's
 * gate / up / down are PRICHS_CKPT_EXPERT0 + 3e + 0 / 1 / 2. */
enum {
  PRICHS_CKPT_INPUT_NORM = 0,
  PRICHS_CKPT_Q_PROJ = 1,
  PRICHS_CKPT_K_PROJ = 2,
  PRICHS_CKPT_V_PROJ = 3,
  PRICHS_CKPT_OUT_PROJ = 4,
  PRICHS_CKPT_POST_ATTN_NORM = 5,
  PRICHS_CKPT_ROUTER = 6,
  PRICHS_CKPT_SHARED_GATE = 7,
  PRICHS_CKPT_SHARED_UP = 8,
  PRICHS_CKPT_SHARED_DOWN = 9,
  PRICHS_CKPT_EXPERT0 = 10
};
/* Parameter index of `slot` in block `layer` of a model with E routed
 * experts: 2 + layer * (10 + 3E) + slot (model.rs:557-562, 1083-1087);
 * (size_t)-1 when slot >= 10 + 3E. */
size_t prichs_checkpoint_block_param(size_t layer, size_t E, size_t slot);

/* Uploads the MoE of block `layer` (router, shared expert, routed experts)
 * into an engine created with the file's d, f, E and n_shared = 1 (the
 * reference's layer, moe.rs:61); every length is checked against the engine
 * first.  The aux-free router bias is not a parameter and is not in the
 * file (moe.rs:60; model.rs:312-338): router_bias f32 [E] (host) or NULL =
 * zeros, as a freshly built layer has (moe.rs:75).  Synchronous. */
int prichs_moe_engine_upload_checkpoint(prichs_moe_engine *eng, const prichs_checkpoint *ck,
                                        size_t layer, const float *router_bias);
/* The same for a block engine: both norms, the attention projections and
 * the MoE of block `layer`.  Synchronous. */
int prichs_block_engine_upload_checkpoint(prichs_block_engine *eng, const prichs_checkpoint *ck,
                                          size_t layer, const float *router_bias);

/* ---------------------------------------------------------------------- */
/* 6. General f32 GEMMs: the GPU dispatch target of prichs-core's CPU ops   */
/*    (crates/prichs-core/src/ops.rs:3, 24-31; crates/prichs-cuda/src/      */
/*    cublas.rs:46-327, re-exported at crates/prichs-cuda/src/lib.rs:6-8)   */
/* ---------------------------------------------------------------------- */

/* Operations, in the reference's (m, k, n) naming (cublas.rs:117, 170, 221):
 *   PRICHS_MATMUL_AB:  a [m, k], b [k, n]  -> c [m, n] = a b
 *   PRICHS_MATMUL_ATB: a [m, k], b [m, n]  -> c [k, n] = a^T b
 *   PRICHS_MATMUL_ABT: a [m, k], b [n, k]  -> c [m, n] = a b^T
 * All row-major f32, any sizes (0 included: c = 0 when the reduction is
 * empty).  f32 products and accumulation on v_mfma_f32_16x16x4f32. */
enum { PRICHS_MATMUL_AB = 0, PRICHS_MATMUL_ATB = 1, PRICHS_MATMUL_ABT = 2 };

/* Device pointers, enqueued on `stream`; c is overwritten. */
int prichs_matmul_f32(int op, const float *a, const float *b, float *c, size_t m,
                      size_t k, size_t n, void *stream);

/* GpuWorkspace (cublas.rs:46-115): three device slabs for A, B and C, sized in
 * bytes; 0 selects the reference's sizes (16 MB, 32 MB, 16 MB,
 * cublas.rs:77-84).  The workspace belongs to the device current at
 * creation.  Calls on one handle are serialised by a lock of its own (the
 * reference hands its workspace out as a Mutex<GpuWorkspace>), so threads may
 * share a handle.  Destroying the process-wide handle of
 * prichs_get_gpu_workspace is refused (PRICHS_ERR_INVALID_ARGUMENT). */
typedef struct prichs_gpu_workspace prichs_gpu_workspace;
int prichs_gpu_workspace_create(size_t a_bytes, size_t b_bytes, size_t c_bytes,
                                prichs_gpu_workspace **out);
int prichs_gpu_workspace_destroy(prichs_gpu_workspace *ws);
/* Slab sizes in bytes (any output pointer may be NULL). */
int prichs_gpu_workspace_slabs(const prichs_gpu_workspace *ws, size_t *a_bytes,
                               size_t *b_bytes, size_t *c_bytes);

/* Host slices in and out, synchronous: H2D into slabs A and B, the product
 * into slab C, D2H, device synchronisation.  Operands larger than their slab
 * fail with PRICHS_ERR_CAPACITY before any copy (the reference's "Matrix
 * dimensions exceed preallocated GPU workspace slabs" bail).
 *   matmul      : c  [m, n] = a [m, k] b [k, n]          (cublas.rs:117-166)
 *   matmul_at_b : dw [k, n] = a [m, k]^T b [m, n]         (cublas.rs:170-219)
 *   matmul_a_bt : dx [m, n] = dy [m, k] w [n, k]^T        (cublas.rs:221-268)
 * dw and dx are overwritten, like the reference's GPU path (beta = 0); the
 * reference's CPU matmul_at_b instead adds to dw (ops.rs:72-80). */
int prichs_gpu_workspace_matmul(prichs_gpu_workspace *ws, const float *a,
                                const float *b, float *c, size_t m, size_t k,
                                size_t n);
int prichs_gpu_workspace_matmul_at_b(prichs_gpu_workspace *ws, const float *a,
                                     const float *b, float *dw, size_t m, size_t k,
                                     size_t n);
int prichs_gpu_workspace_matmul_a_bt(prichs_gpu_workspace *ws, const float *dy,
                                     const float *w, float *dx, size_t m, size_t k,
                                     size_t n);

/* get_gpu_workspace (cublas.rs:283-300): the process-wide workspace with the
 * reference's slab sizes, created on first use on the then-current device;
 * NULL (with the reason in prichs_last_error) if that creation failed, and
 * every later call then returns NULL too, as the reference's Lazy does. */
prichs_gpu_workspace *prichs_get_gpu_workspace(void);

/* matmul_gpu / matmul_at_b_gpu / matmul_a_bt_gpu (cublas.rs:302-327): the
 * workspace methods above on the process-wide workspace, serialised by one
 * mutex (the reference's Mutex<GpuWorkspace>).  Without a workspace they
 * return PRICHS_ERR_HIP ("GPU workspace unavailable"), the status on which
 * prichs-core falls back to its CPU loop (ops.rs:27-31). */
int prichs_matmul_gpu(const float *a, const float *b, float *c, size_t m, size_t k,
                      size_t n);
int prichs_matmul_at_b_gpu(const float *a, const float *b, float *dw, size_t m,
                           size_t k, size_t n);
int prichs_matmul_a_bt_gpu(const float *dy, const float *w, float *dx, size_t m,
                           size_t k, size_t n);

/* ---------------------------------------------------------------------- */
/* 7. MoE layer forward that allocates nothing                             */
/* ---------------------------------------------------------------------- */

/* No counterpart in the reference: an entry point for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  It computes prichs_moe_engine_forward
 * (same kernels, same results) without an engine: the caller passes x [T, d]
 * of `dtype`, w_router f32 [d, E], router_bias f32 [E], the packed weights of
 * the n_shared + E experts in the grouped GEMMs' group order (routed 0..E-1,
 * then the shared expert; one prichs_pack_gate_up / prichs_pack_down block
 * each, prichs_packed_gate_up_elems / prichs_packed_down_elems apart), the
 * optional concept bias and out [T, d] of out_dtype -- all device memory.
 * The intermediates (the engine's workspace for T tokens: logits, top-k,
 * permutation, act [T (k + n_shared), f], y [T (k + n_shared), d], 256-byte
 * aligned pieces) live in a library-owned static device array of
 * PRICHS_NOALLOC_SCRATCH_BYTES per GPU; a T that does not fit fails with
 * PRICHS_ERR_CAPACITY before any GPU work (at d = 1536, f = 1280, E = 8,
 * k = 2 about 1,900 tokens fit).  Nothing is allocated or freed.  Calls on
 * one GPU share the array: two calls that overlap on one GPU (other streams
 * or threads) race on it. */
#define PRICHS_NOALLOC_SCRATCH_BYTES (32u << 20)
int prichs_moe_forward_noalloc(const void *x, size_t T, size_t d, size_t f, size_t E,
                               size_t k, size_t n_shared, int dtype,
                               const float *w_router, const float *router_bias,
                               const void *w_gate_up, const void *w_down,
                               const float *concept_bias, size_t n_concept, void *out,
                               int out_dtype, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* PRICHS_HIP_H */
