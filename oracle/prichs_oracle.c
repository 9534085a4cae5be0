/*
 * prichs_oracle.c -- CPU restatement of PRICHS's MoE feed-forward CPU path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * library in prichs_amd/.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it.  The product never calls it.
 *
 * Every function restates one function of the reference (Rust, prichs-core /
 * prichs-model) and cites it by file:line under the reference tree.  The
 * arithmetic order is kept exactly: each product and each sum is rounded to
 * f32 separately (the file is compiled with -ffp-contract=off; Rust never
 * contracts a*b+c into an FMA), loops run in the reference's order, and the
 * transcendental calls (expf, sqrtf, powf, cosf, sinf) go to the same glibc
 * libm that Rust's f32::{exp,sqrt,powf,cos,sin} resolve to on Linux.
 *
 * Row loops that the reference runs under Rayon (par_chunks_exact_mut over
 * output rows) run here under OpenMP over the same rows: Rayon only splits
 * rows between threads, so the per-element arithmetic order is unchanged.
 *
 * Pinning (what checks each function besides this restatement):
 *   orc_matmul_2d            GEMM known-answer test (engine.rs:2881-2910),
 *                            float64 recomputation, exact small-integer case.
 *   orc_matmul_at_b / orc_matmul_a_bt
 *                            bit-identical to orc_matmul_2d on the transposed
 *                            operand (the same summation order), the GEMM
 *                            KAT's backward-data and -weight products
 *                            (engine.rs:2912-2936), float64 recomputation;
 *                            at_b accumulates into dw (its loop adds).
 *   orc_rms_norm             KAT row [2,2,2,2] -> 1.0 (engine.rs:3041-3053),
 *                            float64 closed form.
 *   orc_swiglu / orc_silu    closed form in float64, silu(0)=0, odd/limit cases.
 *   orc_top_k_gating_unbiased  invariants (distinct, descending, ties -> lower
 *                            index, +0 == -0), brute force over all k-subsets,
 *                            bias changes selection only, NaN cases against an
 *                            independent Python insertion-sort model.
 *   orc_moe_forward          float64 re-assembly of the layer from numpy,
 *                            permutation = stable counting sort, committed
 *                            golden fixture for config 1.
 *   orc_precompute_rope_cache / orc_rope_forward_in_place
 *                            cos=1/sin=0 identity (engine.rs:2970-2972), norm
 *                            preservation, float64 closed form.
 *   orc_attention_forward    float64 causal-softmax attention recomputed in
 *                            numpy (GQA head mapping, RoPE); softmax rows sum
 *                            to 1 and causal zeros (engine.rs:2948-3029);
 *                            row 0 attends only to itself.
 *   orc_block_forward        float64 re-assembly of the block from the pinned
 *                            pieces (RMSNorm, attention, MoE, residuals).
 *   orc_moe_backward         central finite differences of the pinned
 *                            forward (<d_out, out>) on small shapes for d_x
 *                            and every weight gradient (dx_weighting = 1);
 *                            dx_weighting = 2 differs only in the routed d_x
 *                            term, by exactly the extra gate-weight factor.
 *   orc_update_aux_free_bias float64 closed form; the update sums to ~0 over
 *                            the experts (sum of counts = k * T); balanced
 *                            routing leaves the bias unchanged; T = 0 no-op.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------------ */
/* GEMM: crates/prichs-core/src/ops.rs:8-61 (CPU branch ops.rs:33-58).        */
/* out[i][j] = (((0 + a[i][0]*b[0][j]) + a[i][1]*b[1][j]) + ...)              */
/* The m == 1 fast path (ops.rs:34-43) has the same per-element order.        */
/* ------------------------------------------------------------------------ */
ORC_API void orc_matmul_2d(const float *a, const float *b, float *out,
                           size_t m, size_t k, size_t n) {
  long long mi;
#pragma omp parallel for schedule(static)
  for (mi = 0; mi < (long long)m; ++mi) {
    const float *a_row = a + (size_t)mi * k;
    float *out_row = out + (size_t)mi * n;
    for (size_t j = 0; j < n; ++j) out_row[j] = 0.0f;
    for (size_t kk = 0; kk < k; ++kk) {
      const float a_val = a_row[kk];
      const float *b_row = b + kk * n;
      for (size_t j = 0; j < n; ++j) {
        float prod = a_val * b_row[j];
        out_row[j] = out_row[j] + prod;
      }
    }
  }
}

/* crates/prichs-core/src/ops.rs:63-83, CPU branch of matmul_at_b: dW[k, n]
 * += A[m, k]^T B[m, n].  For each row i of dW, t ascending, j ascending:
 * dw[i][j] = dw[i][j] + a[t][i] * b[t][j] (product rounded, then the sum).
 * Like the reference's CPU loop it ACCUMULATES into dw (its GPU branch,
 * cublas.rs:170-219, overwrites). */
ORC_API void orc_matmul_at_b(const float *a, const float *b, float *dw,
                             size_t m, size_t k, size_t n) {
  long long ii;
#pragma omp parallel for schedule(static)
  for (ii = 0; ii < (long long)k; ++ii) {
    float *dw_row = dw + (size_t)ii * n;
    for (size_t t = 0; t < m; ++t) {
      const float a_val = a[t * k + (size_t)ii];
      const float *b_row = b + t * n;
      for (size_t j = 0; j < n; ++j) {
        float prod = a_val * b_row[j];
        dw_row[j] = dw_row[j] + prod;
      }
    }
  }
}

/* ops.rs:85-107, CPU branch of matmul_a_bt: dX[m, n] = dY[m, k] W[n, k]^T,
 * each element a sequential dot product from 0 over c ascending (the result
 * overwrites dx). */
ORC_API void orc_matmul_a_bt(const float *dy, const float *w, float *dx,
                             size_t m, size_t k, size_t n) {
  long long mi;
#pragma omp parallel for schedule(static)
  for (mi = 0; mi < (long long)m; ++mi) {
    const float *dy_row = dy + (size_t)mi * k;
    for (size_t j = 0; j < n; ++j) {
      const float *w_row = w + j * k;
      float dot = 0.0f;
      for (size_t c = 0; c < k; ++c) {
        float prod = dy_row[c] * w_row[c];
        dot = dot + prod;
      }
      dx[(size_t)mi * n + j] = dot;
    }
  }
}

/* ------------------------------------------------------------------------ */
/* RMSNorm: crates/prichs-core/src/ops.rs:109-135.                            */
/* sum_sq sequential over the row (Iterator::sum), rms = sqrt(ss/d + eps),    */
/* inv = 1/rms, out = (x*inv)*w.                                              */
/* ------------------------------------------------------------------------ */
ORC_API void orc_rms_norm(const float *x, const float *w, float *out,
                          size_t rows, size_t d, float eps) {
  long long r;
#pragma omp parallel for schedule(static)
  for (r = 0; r < (long long)rows; ++r) {
    const float *row = x + (size_t)r * d;
    float *orow = out + (size_t)r * d;
    float sum_sq = 0.0f;
    for (size_t c = 0; c < d; ++c) {
      float sq = row[c] * row[c];
      sum_sq = sum_sq + sq;
    }
    float rms = sqrtf(sum_sq / (float)d + eps);
    float inv_rms = 1.0f / rms;
    for (size_t c = 0; c < d; ++c) {
      float t = row[c] * inv_rms;
      orow[c] = t * w[c];
    }
  }
}

/* silu: crates/prichs-core/src/ops.rs:137-140.  x / (1 + exp(-x)). */
ORC_API float orc_silu(float x) {
  float den = 1.0f + expf(-x);
  return x / den;
}

/* SwiGLU: crates/prichs-core/src/ops.rs:142-159.  out = silu(g) * u. */
ORC_API void orc_swiglu(const float *g, const float *u, float *out, size_t n) {
  long long i;
#pragma omp parallel for schedule(static)
  for (i = 0; i < (long long)n; ++i) out[i] = orc_silu(g[i]) * u[i];
}

/* add_tensors: crates/prichs-core/src/ops.rs:250-267. */
ORC_API void orc_add_tensors(const float *a, const float *b, float *out,
                             size_t n) {
  long long i;
#pragma omp parallel for schedule(static)
  for (i = 0; i < (long long)n; ++i) out[i] = a[i] + b[i];
}

/* ------------------------------------------------------------------------ */
/* top_k_gating_unbiased: crates/prichs-core/src/ops.rs:219-248.              */
/*                                                                            */
/* Selection: slice::sort_by on (index, routing_logit) with comparator        */
/* b.partial_cmp(a).unwrap_or(Equal) -- a stable descending sort.  For the    */
/* slice lengths used here (E <= 20) Rust's stable sort is an insertion sort  */
/* that inserts v[i] leftwards while is_less(v[i], v[j-1]) holds, where       */
/* is_less(x, y) == (compare(x, y) == Less) == (x.val > y.val).  A NaN never  */
/* compares Less, so the insertion sort below reproduces the reference on     */
/* NaN inputs too; on non-NaN inputs it is the stable descending order (ties  */
/* keep ascending index, +0 and -0 compare equal).                            */
/*                                                                            */
/* Weights: softmax over the RAW logits of the selected experts in slot      */
/* order: m = fold(-inf, f32::max), e_i = exp(raw_i - m), s = sequential sum, */
/* inv = 1/(s + 1e-9), w_i = e_i * inv.                                       */
/* ------------------------------------------------------------------------ */
#define ORC_MAX_E 256
ORC_API int orc_top_k_gating_unbiased(const float *raw, const float *adj,
                                      size_t E, size_t k, int32_t *idx_out,
                                      float *w_out) {
  if (E == 0 || E > ORC_MAX_E || k > E) return -1;
  int32_t ord[ORC_MAX_E];
  float val[ORC_MAX_E];
  for (size_t i = 0; i < E; ++i) {
    ord[i] = (int32_t)i;
    val[i] = adj[i];
  }
  for (size_t i = 1; i < E; ++i) {
    int32_t oi = ord[i];
    float vi = val[i];
    size_t j = i;
    while (j > 0 && (vi > val[j - 1])) { /* is_less(v[i], v[j-1]) */
      ord[j] = ord[j - 1];
      val[j] = val[j - 1];
      --j;
    }
    ord[j] = oi;
    val[j] = vi;
  }
  float max_val = -INFINITY;
  for (size_t s = 0; s < k; ++s) max_val = fmaxf(max_val, raw[ord[s]]);
  float e_buf[ORC_MAX_E];
  float sum_exp = 0.0f;
  for (size_t s = 0; s < k; ++s) {
    float diff = raw[ord[s]] - max_val;
    float e = expf(diff);
    e_buf[s] = e;
    sum_exp = sum_exp + e;
  }
  float inv_sum = 1.0f / (sum_exp + 1e-9f);
  for (size_t s = 0; s < k; ++s) {
    idx_out[s] = ord[s];
    w_out[s] = e_buf[s] * inv_sum;
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Router + gating for all tokens: crates/prichs-model/src/moe.rs:113-142.    */
/* raw = x @ W_router (ops.rs GEMM order); adj = (raw + bias[e]) (+ c[e] for  */
/* e < n_concept); per token top_k_gating_unbiased(raw, adj, k).              */
/* ------------------------------------------------------------------------ */
ORC_API int orc_route(const float *x, const float *w_router,
                      const float *router_bias, const float *concept_bias,
                      size_t n_concept, size_t T, size_t d, size_t E, size_t k,
                      float *logits_out, int32_t *sel_out, float *gw_out) {
  if (E == 0 || E > ORC_MAX_E || k > E) return -1;
  orc_matmul_2d(x, w_router, logits_out, T, d, E);
  long long t;
  int bad = 0;
#pragma omp parallel for schedule(static) reduction(| : bad)
  for (t = 0; t < (long long)T; ++t) {
    const float *raw = logits_out + (size_t)t * E;
    float adj[ORC_MAX_E];
    for (size_t e = 0; e < E; ++e) {
      float logit = raw[e] + router_bias[e];
      if (concept_bias != NULL && e < n_concept) logit = logit + concept_bias[e];
      adj[e] = logit;
    }
    bad |= orc_top_k_gating_unbiased(raw, adj, E, k, sel_out + (size_t)t * k,
                                     gw_out + (size_t)t * k);
  }
  return bad ? -1 : 0;
}

/* ------------------------------------------------------------------------ */
/* Token binning: crates/prichs-model/src/moe.rs:121, 137-141, 149-153.       */
/* expert_assignments[e] gets (t, w) for t ascending; experts are visited in  */
/* ascending order.  Flattened: offsets[E+1], row_token[T*k], row_weight,     */
/* and the inverse map token_row[t*k + slot].                                 */
/* ------------------------------------------------------------------------ */
ORC_API void orc_bin_tokens(const int32_t *sel, const float *gw, size_t T,
                            size_t E, size_t k, int32_t *offsets,
                            int32_t *row_token, float *row_weight,
                            int32_t *token_row) {
  size_t counts[ORC_MAX_E];
  for (size_t e = 0; e < E; ++e) counts[e] = 0;
  for (size_t i = 0; i < T * k; ++i) counts[sel[i]]++;
  offsets[0] = 0;
  for (size_t e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + (int32_t)counts[e];
  size_t cursor[ORC_MAX_E];
  for (size_t e = 0; e < E; ++e) cursor[e] = (size_t)offsets[e];
  for (size_t t = 0; t < T; ++t) {
    for (size_t s = 0; s < k; ++s) {
      int32_t e = sel[t * k + s];
      size_t r = cursor[e]++;
      row_token[r] = (int32_t)t;
      row_weight[r] = gw[t * k + s];
      if (token_row) token_row[t * k + s] = (int32_t)r;
    }
  }
}

/* Expert::forward shape: G = X Wg, U = X Wu, A = swiglu(G, U), Y = A Wd.
 * crates/prichs-model/src/moe.rs:22-28 and 166-170. */
static int orc_expert_ffn(const float *xin, size_t m, size_t d, size_t f,
                          const float *wg, const float *wu, const float *wd,
                          float *y) {
  float *g = (float *)malloc(sizeof(float) * m * f);
  float *u = (float *)malloc(sizeof(float) * m * f);
  if (!g || !u) {
    free(g);
    free(u);
    return -1;
  }
  orc_matmul_2d(xin, wg, g, m, d, f);
  orc_matmul_2d(xin, wu, u, m, d, f);
  orc_swiglu(g, u, g, m * f);
  orc_matmul_2d(g, wd, y, m, f, d);
  free(g);
  free(u);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* MoELayer::update_aux_free_bias: crates/prichs-model/src/moe.rs:228-245.    */
/* target = top_k / E; per expert actual = counts[i] / total_tokens,          */
/* diff = target - actual, bias[i] += gamma * diff (all f32, usize -> f32     */
/* conversions rounded to nearest).  Returns without change when             */
/* total_tokens == 0 or E == 0.  The reference's training step passes the    */
/* per-expert assignment counts of the last batch and its token count         */
/* (model.rs:1541-1547).                                                      */
/* ------------------------------------------------------------------------ */
ORC_API void orc_update_aux_free_bias(float *bias, const int64_t *counts, size_t E,
                                      size_t top_k, size_t total_tokens, float gamma) {
  if (total_tokens == 0 || E == 0) return;
  const float target = (float)top_k / (float)E;
  for (size_t i = 0; i < E; ++i) {
    const float actual = (float)counts[i] / (float)total_tokens;
    const float diff = target - actual;
    bias[i] += gamma * diff;
  }
}

/* ------------------------------------------------------------------------ */
/* MoELayer::forward_train: crates/prichs-model/src/moe.rs:93-212.            */
/*                                                                            */
/* 1. shared expert on all rows (moe.rs:103-106);                             */
/* 2. router logits + per-token gating (moe.rs:113-142);                      */
/* 3. total_out = shared_out (moe.rs:146);                                    */
/* 4. for e ascending with a non-empty bin: gather rows, expert FFN, then     */
/*    out[t] += w * y row by row (moe.rs:149-184).                            */
/*                                                                            */
/* Weights: gate/up [d,f], down [f,d] row-major (moe.rs:16-18); the shared    */
/* expert comes first in the arrays (n_shared = 0 or 1), then routed 0..E-1.  */
/* Optional outputs (NULL to skip): logits [T,E], sel [T,k], gw [T,k],        */
/* offsets [E+1], row_token [T*k], row_weight [T*k], token_row [T*k].         */
/* ------------------------------------------------------------------------ */
ORC_API int orc_moe_forward(const float *x, size_t T, size_t d, size_t f,
                            size_t E, size_t k, size_t n_shared,
                            const float *w_router, const float *router_bias,
                            const float *concept_bias, size_t n_concept,
                            const float *const *w_gate,
                            const float *const *w_up,
                            const float *const *w_down, float *out,
                            float *logits, int32_t *sel, float *gw,
                            int32_t *offsets, int32_t *row_token,
                            float *row_weight, int32_t *token_row) {
  if (E == 0 || E > ORC_MAX_E || k > E || n_shared > 1) return -1;
  int rc = 0;
  float *lg = logits ? logits : (float *)malloc(sizeof(float) * (T * E + 1));
  int32_t *sl = sel ? sel : (int32_t *)malloc(sizeof(int32_t) * (T * k + 1));
  float *gwt = gw ? gw : (float *)malloc(sizeof(float) * (T * k + 1));
  int32_t *off = offsets ? offsets : (int32_t *)malloc(sizeof(int32_t) * (E + 1));
  int32_t *rt = row_token ? row_token : (int32_t *)malloc(sizeof(int32_t) * (T * k + 1));
  float *rw = row_weight ? row_weight : (float *)malloc(sizeof(float) * (T * k + 1));
  if (!lg || !sl || !gwt || !off || !rt || !rw) rc = -1;

  /* 1. shared expert, written straight into out (total_out = shared_out). */
  if (rc == 0) {
    if (n_shared == 1) {
      rc = orc_expert_ffn(x, T, d, f, w_gate[0], w_up[0], w_down[0], out);
    } else {
      memset(out, 0, sizeof(float) * T * d);
    }
  }
  /* 2. routing. */
  if (rc == 0)
    rc = orc_route(x, w_router, router_bias, concept_bias, n_concept, T, d, E, k,
                   lg, sl, gwt);
  if (rc == 0) orc_bin_tokens(sl, gwt, T, E, k, off, rt, rw, token_row);

  /* 3./4. routed experts in ascending order, scatter-add row by row. */
  for (size_t e = 0; rc == 0 && e < E; ++e) {
    size_t n_tok = (size_t)(off[e + 1] - off[e]);
    if (n_tok == 0) continue;
    float *xb = (float *)malloc(sizeof(float) * n_tok * d);
    float *yb = (float *)malloc(sizeof(float) * n_tok * d);
    if (!xb || !yb) {
      free(xb);
      free(yb);
      rc = -1;
      break;
    }
    for (size_t i = 0; i < n_tok; ++i)
      memcpy(xb + i * d, x + (size_t)rt[off[e] + i] * d, sizeof(float) * d);
    rc = orc_expert_ffn(xb, n_tok, d, f, w_gate[n_shared + e],
                        w_up[n_shared + e], w_down[n_shared + e], yb);
    if (rc == 0) {
      /* Rows of one bin belong to distinct tokens, so rows can be updated in
       * parallel without changing any element's order of additions. */
      long long i;
#pragma omp parallel for schedule(static)
      for (i = 0; i < (long long)n_tok; ++i) {
        size_t r = (size_t)off[e] + (size_t)i;
        float wgt = rw[r];
        float *orow = out + (size_t)rt[r] * d;
        const float *yrow = yb + (size_t)i * d;
        for (size_t c = 0; c < d; ++c) {
          float prod = wgt * yrow[c];
          orow[c] = orow[c] + prod;
        }
      }
    }
    free(xb);
    free(yb);
  }

  if (!logits) free(lg);
  if (!sel) free(sl);
  if (!gw) free(gwt);
  if (!offsets) free(off);
  if (!row_token) free(rt);
  if (!row_weight) free(rw);
  return rc;
}

/* ------------------------------------------------------------------------ */
/* MoE backward: the reference's training step (model.rs:1474-1561) through   */
/* GpuModelEngine::gpu_moe_backward_expert / _shared / _router                */
/* (engine.rs:2242-2789), its kernels (kernels.cu:459-480, 926-991) and the   */
/* router VJP moe_router_unbiased_backward (backward.rs:269-287), in f32 with */
/* one fixed order of additions.                                              */
/*                                                                            */
/* Forward (recomputed here): routing and binning as orc_moe_forward; per     */
/* expert G = X Wg, U = X Wu, A = silu(G) U, Y = A Wd (Y before the gate      */
/* weight, the reference's stashed expert output).                            */
/* Per routed expert e ascending, rows r of its bin (token t, weight w):      */
/*   dY[r] = w * d_out[t]                          (gather_weighted)          */
/*   s[r]  = sum_c Y[r][c] * d_out[t][c]           (router_dot)               */
/*   dWd  += A^T dY;  dA = dY Wd^T                                            */
/*   sig = 1/(1+exp(-g)); dU = dA*silu(g); dG = (dA*u)*(sig*(1+g*(1-sig)))    */
/*   dWg  += X^T dG;  dWu += X^T dU                                           */
/*   d_x[t] += w * (dG Wg^T + dU Wu^T)[r]          (scatter_add_grad)         */
/* The reference's gather already scaled dY by w, so its scatter applies the  */
/* gate weight to the routed input gradient a second time; dx_weighting = 2   */
/* restates that, dx_weighting = 1 drops the second factor (the chain rule).  */
/* Weight gradients do not depend on it.                                      */
/* Shared expert (weight 1, all T rows): the same with dY = d_out; its two    */
/* input-gradient GEMMs accumulate into d_x one after the other.              */
/* Router, per token: d_w[j] = s of its j-th selected expert;                 */
/*   ws = sum_j g_j d_w[j];  d_logits[t][e_j] = g_j * (d_w[j] - ws), else 0;  */
/*   dW_router += x^T d_logits;  d_x += d_logits W_router^T.                  */
/* d_x is overwritten (the reference clears it first); every dW is added to   */
/* (cuBLAS beta = 1): dW += (sum over rows ascending of the products).        */
/* Order of the d_x additions: routed experts ascending (rows ascending),     */
/* shared gate then up products, router.                                      */
/* ------------------------------------------------------------------------ */

/* dw[i][j] += sum_r a[r][i] * b[r][j] (r ascending), a [m, p], b [m, q]. */
static void orc_accum_at_b(const float *a, const float *b, float *dw, size_t m, size_t p,
                           size_t q) {
  long long i;
#pragma omp parallel for schedule(static)
  for (i = 0; i < (long long)p; ++i) {
    float *acc = (float *)calloc(q, sizeof(float));
    if (!acc) continue;
    for (size_t r = 0; r < m; ++r) {
      const float av = a[r * p + (size_t)i];
      const float *brow = b + r * q;
      for (size_t j = 0; j < q; ++j) {
        float prod = av * brow[j];
        acc[j] = acc[j] + prod;
      }
    }
    float *drow = dw + (size_t)i * q;
    for (size_t j = 0; j < q; ++j) drow[j] = drow[j] + acc[j];
    free(acc);
  }
}

/* out[r][i] = sum_j a[r][j] * w[i][j] (j ascending): a [m, q], w [p, q]. */
static void orc_matmul_bt(const float *a, const float *w, float *out, size_t m, size_t q,
                          size_t p) {
  long long r;
#pragma omp parallel for schedule(static)
  for (r = 0; r < (long long)m; ++r) {
    const float *arow = a + (size_t)r * q;
    for (size_t i = 0; i < p; ++i) {
      const float *wrow = w + i * q;
      float acc = 0.0f;
      for (size_t j = 0; j < q; ++j) {
        float prod = arow[j] * wrow[j];
        acc = acc + prod;
      }
      out[(size_t)r * p + i] = acc;
    }
  }
}

/* SwiGLU backward, kernels.cu:459-480 in f32 with expf. */
static void orc_swiglu_backward(const float *da, const float *g, const float *u, float *dg,
                                float *du, size_t n) {
  long long i;
#pragma omp parallel for schedule(static)
  for (i = 0; i < (long long)n; ++i) {
    const float gv = g[i], uv = u[i], dy = da[i];
    const float sig = 1.0f / (1.0f + expf(-gv));
    const float silu = gv * sig;
    const float dsilu = sig * (1.0f + gv * (1.0f - sig));
    du[i] = dy * silu;
    const float dyu = dy * uv;
    dg[i] = dyu * dsilu;
  }
}

/* One expert's backward on m rows of xin (rows of d_out given by dy, already
 * weighted).  Accumulates dWg, dWu, dWd; writes dX [m, d] = dG Wg^T + dU Wu^T
 * as two products (dxg, dxu) and Y [m, d] when y != NULL. */
static int orc_expert_backward(const float *xin, const float *dy, size_t m, size_t d, size_t f,
                               const float *wg, const float *wu, const float *wd, float *dwg,
                               float *dwu, float *dwd, float *dxg, float *dxu, float *y) {
  float *g = (float *)malloc(sizeof(float) * m * f);
  float *u = (float *)malloc(sizeof(float) * m * f);
  float *a = (float *)malloc(sizeof(float) * m * f);
  float *da = (float *)malloc(sizeof(float) * m * f);
  int rc = (g && u && a && da) ? 0 : -1;
  if (rc == 0) {
    orc_matmul_2d(xin, wg, g, m, d, f);
    orc_matmul_2d(xin, wu, u, m, d, f);
    orc_swiglu(g, u, a, m * f);
    if (y) orc_matmul_2d(a, wd, y, m, f, d);
    orc_accum_at_b(a, dy, dwd, m, f, d);    /* dWd [f, d] += A^T dY */
    orc_matmul_bt(dy, wd, da, m, d, f);     /* dA = dY Wd^T          */
    orc_swiglu_backward(da, g, u, g, u, m * f); /* g <- dG, u <- dU   */
    orc_accum_at_b(xin, g, dwg, m, d, f);   /* dWg [d, f] += X^T dG  */
    orc_accum_at_b(xin, u, dwu, m, d, f);   /* dWu [d, f] += X^T dU  */
    orc_matmul_bt(g, wg, dxg, m, f, d);     /* dG Wg^T               */
    orc_matmul_bt(u, wu, dxu, m, f, d);     /* dU Wu^T               */
  }
  free(g);
  free(u);
  free(a);
  free(da);
  return rc;
}

ORC_API int orc_moe_backward(const float *x, const float *d_out, size_t T, size_t d, size_t f,
                             size_t E, size_t k, const float *w_router,
                             const float *router_bias, const float *concept_bias,
                             size_t n_concept, const float *const *w_gate,
                             const float *const *w_up, const float *const *w_down,
                             int dx_weighting, float *d_x, float *dw_router,
                             float *const *dw_gate, float *const *dw_up,
                             float *const *dw_down) {
  if (E == 0 || E > ORC_MAX_E || k == 0 || k > E || (dx_weighting != 1 && dx_weighting != 2))
    return -1;
  int rc = 0;
  float *lg = (float *)malloc(sizeof(float) * (T * E + 1));
  int32_t *sl = (int32_t *)malloc(sizeof(int32_t) * (T * k + 1));
  float *gw = (float *)malloc(sizeof(float) * (T * k + 1));
  int32_t *off = (int32_t *)malloc(sizeof(int32_t) * (E + 1));
  int32_t *rt = (int32_t *)malloc(sizeof(int32_t) * (T * k + 1));
  float *rw = (float *)malloc(sizeof(float) * (T * k + 1));
  int32_t *tr = (int32_t *)malloc(sizeof(int32_t) * (T * k + 1));
  float *scal = (float *)calloc(T * E + 1, sizeof(float)); /* s per (token, expert) */
  float *dlog = (float *)calloc(T * E + 1, sizeof(float));
  if (!lg || !sl || !gw || !off || !rt || !rw || !tr || !scal || !dlog) rc = -1;
  if (rc == 0)
    rc = orc_route(x, w_router, router_bias, concept_bias, n_concept, T, d, E, k, lg, sl, gw);
  if (rc == 0) orc_bin_tokens(sl, gw, T, E, k, off, rt, rw, tr);
  if (rc == 0) memset(d_x, 0, sizeof(float) * T * d);

  /* Routed experts, ascending. */
  for (size_t e = 0; rc == 0 && e < E; ++e) {
    const size_t m = (size_t)(off[e + 1] - off[e]);
    if (m == 0) continue;
    float *xb = (float *)malloc(sizeof(float) * m * d);
    float *dy = (float *)malloc(sizeof(float) * m * d);
    float *y = (float *)malloc(sizeof(float) * m * d);
    float *dxg = (float *)malloc(sizeof(float) * m * d);
    float *dxu = (float *)malloc(sizeof(float) * m * d);
    if (!xb || !dy || !y || !dxg || !dxu) rc = -1;
    for (size_t i = 0; rc == 0 && i < m; ++i) {
      const size_t r = (size_t)off[e] + i, t = (size_t)rt[r];
      memcpy(xb + i * d, x + t * d, sizeof(float) * d);
      for (size_t c = 0; c < d; ++c) dy[i * d + c] = rw[r] * d_out[t * d + c];
    }
    if (rc == 0)
      rc = orc_expert_backward(xb, dy, m, d, f, w_gate[1 + e], w_up[1 + e], w_down[1 + e],
                               dw_gate[1 + e], dw_up[1 + e], dw_down[1 + e], dxg, dxu, y);
    for (size_t i = 0; rc == 0 && i < m; ++i) {
      const size_t r = (size_t)off[e] + i, t = (size_t)rt[r];
      float s = 0.0f;
      for (size_t c = 0; c < d; ++c) {
        float prod = y[i * d + c] * d_out[t * d + c];
        s = s + prod;
      }
      scal[t * E + e] = s;
      const float wx = dx_weighting == 2 ? rw[r] : 1.0f;
      for (size_t c = 0; c < d; ++c) {
        const float sum = dxg[i * d + c] + dxu[i * d + c];
        const float val = wx * sum;
        d_x[t * d + c] = d_x[t * d + c] + val;
      }
    }
    free(xb);
    free(dy);
    free(y);
    free(dxg);
    free(dxu);
  }

  /* Shared expert on all rows, weight 1. */
  if (rc == 0) {
    float *dxg = (float *)malloc(sizeof(float) * T * d);
    float *dxu = (float *)malloc(sizeof(float) * T * d);
    if (!dxg || !dxu) rc = -1;
    if (rc == 0)
      rc = orc_expert_backward(x, d_out, T, d, f, w_gate[0], w_up[0], w_down[0], dw_gate[0],
                               dw_up[0], dw_down[0], dxg, dxu, NULL);
    if (rc == 0) {
      for (size_t i = 0; i < T * d; ++i) d_x[i] = d_x[i] + dxg[i];
      for (size_t i = 0; i < T * d; ++i) d_x[i] = d_x[i] + dxu[i];
    }
    free(dxg);
    free(dxu);
  }

  /* Router VJP per token, then its two products. */
  if (rc == 0) {
    for (size_t t = 0; t < T; ++t) {
      const int32_t *idx = sl + t * k;
      const float *g = gw + t * k;
      float ws = 0.0f;
      for (size_t j = 0; j < k; ++j) {
        float prod = g[j] * scal[t * E + (size_t)idx[j]];
        ws = ws + prod;
      }
      for (size_t j = 0; j < k; ++j) {
        const float diff = scal[t * E + (size_t)idx[j]] - ws;
        dlog[t * E + (size_t)idx[j]] = g[j] * diff;
      }
    }
    orc_accum_at_b(x, dlog, dw_router, T, d, E); /* dW_router [d, E] += x^T d_logits */
    float *dxr = (float *)malloc(sizeof(float) * T * d);
    if (!dxr) {
      rc = -1;
    } else {
      /* d_logits W_router^T: W_router is [d, E], so row c of it is w_router[c][:]. */
      orc_matmul_bt(dlog, w_router, dxr, T, E, d);
      for (size_t i = 0; i < T * d; ++i) d_x[i] = d_x[i] + dxr[i];
      free(dxr);
    }
  }
  free(lg);
  free(sl);
  free(gw);
  free(off);
  free(rt);
  free(rw);
  free(tr);
  free(scal);
  free(dlog);
  return rc;
}

/* ------------------------------------------------------------------------ */
/* RoPE cache: crates/prichs-core/src/backward.rs:136-157.                    */
/* freq_i = 1 / theta^((2i)/hd) (f32 powf), angle = (t as f32) * freq_i.      */
/* ------------------------------------------------------------------------ */
ORC_API void orc_precompute_rope_cache(size_t max_seq_len, size_t head_dim,
                                       float theta, float *cos_cache,
                                       float *sin_cache) {
  size_t half = head_dim / 2;
  for (size_t i = 0; i < half; ++i) {
    float exponent = (float)(2 * i) / (float)head_dim;
    float freq = 1.0f / powf(theta, exponent);
    for (size_t t = 0; t < max_seq_len; ++t) {
      float angle = (float)t * freq;
      size_t off = t * half + i;
      cos_cache[off] = cosf(angle);
      sin_cache[off] = sinf(angle);
    }
  }
}

/* RoPE rotation: crates/prichs-core/src/backward.rs:160-188.
 * Interleaved pairs (2i, 2i+1) at position t + pos_offset. */
ORC_API void orc_rope_forward_in_place(float *tensor, const float *cos_cache,
                                       const float *sin_cache, size_t seq_len,
                                       size_t n_heads, size_t head_dim,
                                       size_t pos_offset) {
  size_t half = head_dim / 2;
  for (size_t t = 0; t < seq_len; ++t) {
    size_t trig = (t + pos_offset) * half;
    for (size_t h = 0; h < n_heads; ++h) {
      size_t base = (t * n_heads + h) * head_dim;
      for (size_t i = 0; i < half; ++i) {
        float c = cos_cache[trig + i];
        float s = sin_cache[trig + i];
        float q0 = tensor[base + 2 * i];
        float q1 = tensor[base + 2 * i + 1];
        float a0 = q0 * c, b0 = q1 * s;
        float a1 = q0 * s, b1 = q1 * c;
        tensor[base + 2 * i] = a0 - b0;
        tensor[base + 2 * i + 1] = a1 + b1;
      }
    }
  }
}

/* ------------------------------------------------------------------------ */
/* Self-attention of one sequence: crates/prichs-model/src/attention.rs:56-176 */
/*                                                                            */
/* q = x Wq, k = x Wk, v = x Wv (ops.rs GEMM order); RoPE on q (Hq heads) and */
/* k (Hkv heads) at positions t + pos_offset; per head h with kv head         */
/* h / (Hq / Hkv):                                                            */
/*   score[i][j] = (sum_d q[i][d] k[j][d]) * scale, j <= i, d ascending,      */
/*     scale = 1 / sqrt(hd) in f32;                                           */
/*   softmax over j <= i: m = fold(-inf, max), e = exp(s - m), s = sum e      */
/*     (j ascending), p = e * (1 / max(s, 1e-9));                             */
/*   head_out[i][d] = sum over j ascending of p[j] * v[j][d] (product, then  */
/*     sum).                                                                  */
/* concat heads along columns (head h at h*hd), out = concat Wo.              */
/* Requires Hq * hd == d (attention.rs indexes q rows with hidden_dim).       */
/* attn_concat [S, d] may be NULL.                                            */
/* ------------------------------------------------------------------------ */
ORC_API int orc_attention_forward(const float *x, size_t S, size_t d, size_t Hq,
                                  size_t Hkv, size_t hd, const float *wq,
                                  const float *wk, const float *wv,
                                  const float *wo, const float *cos_cache,
                                  const float *sin_cache, size_t pos_offset,
                                  float *out, float *attn_concat) {
  if (Hq == 0 || Hkv == 0 || Hq % Hkv || Hq * hd != d || hd % 2) return -1;
  const size_t kvw = Hkv * hd;
  float *q = (float *)malloc(sizeof(float) * S * d);
  float *k = (float *)malloc(sizeof(float) * S * kvw);
  float *v = (float *)malloc(sizeof(float) * S * kvw);
  float *cat = attn_concat ? attn_concat : (float *)malloc(sizeof(float) * S * d);
  if (!q || !k || !v || !cat) {
    free(q);
    free(k);
    free(v);
    if (!attn_concat) free(cat);
    return -1;
  }
  orc_matmul_2d(x, wq, q, S, d, d);
  orc_matmul_2d(x, wk, k, S, d, kvw);
  orc_matmul_2d(x, wv, v, S, d, kvw);
  orc_rope_forward_in_place(q, cos_cache, sin_cache, S, Hq, hd, pos_offset);
  orc_rope_forward_in_place(k, cos_cache, sin_cache, S, Hkv, hd, pos_offset);
  const float scale = 1.0f / sqrtf((float)hd);
  const size_t group = Hq / Hkv;
  int bad = 0;
  long long h;
#pragma omp parallel for schedule(dynamic) reduction(| : bad)
  for (h = 0; h < (long long)Hq; ++h) {
    const size_t kvh = (size_t)h / group;
    float *row = (float *)malloc(sizeof(float) * (S ? S : 1));
    float *acc = (float *)malloc(sizeof(float) * hd);
    if (!row || !acc) {
      bad = 1;
      free(row);
      free(acc);
      continue;
    }
    for (size_t i = 0; i < S; ++i) {
      const float *qr = q + i * d + (size_t)h * hd;
      for (size_t j = 0; j <= i; ++j) {
        const float *kr = k + j * kvw + kvh * hd;
        float dot = 0.0f;
        for (size_t c = 0; c < hd; ++c) {
          float p = qr[c] * kr[c];
          dot = dot + p;
        }
        row[j] = dot * scale;
      }
      float mx = -INFINITY;
      for (size_t j = 0; j <= i; ++j) mx = fmaxf(mx, row[j]);
      float sum = 0.0f;
      for (size_t j = 0; j <= i; ++j) {
        float e = expf(row[j] - mx);
        row[j] = e;
        sum = sum + e;
      }
      const float inv = 1.0f / fmaxf(sum, 1e-9f);
      for (size_t j = 0; j <= i; ++j) row[j] = row[j] * inv;
      for (size_t c = 0; c < hd; ++c) acc[c] = 0.0f;
      for (size_t j = 0; j <= i; ++j) {
        const float *vr = v + j * kvw + kvh * hd;
        const float w = row[j];
        for (size_t c = 0; c < hd; ++c) {
          float p = w * vr[c];
          acc[c] = acc[c] + p;
        }
      }
      memcpy(cat + i * d + (size_t)h * hd, acc, sizeof(float) * hd);
    }
    free(row);
    free(acc);
  }
  if (!bad) orc_matmul_2d(cat, wo, out, S, d, d);
  free(q);
  free(k);
  free(v);
  if (!attn_concat) free(cat);
  return bad ? -1 : 0;
}

/* ------------------------------------------------------------------------ */
/* PrichsBlock::forward_with_rope: crates/prichs-model/src/block.rs:50-68,    */
/* for `batch` independent sequences of seq_len rows (the block has no batch  */
/* dimension; rows of different sequences never meet in attention, and the    */
/* per-token RMSNorm / MoE / residual steps are row-wise):                     */
/*   n1 = rms_norm(x, input_norm); x1 = x + Attn(n1);                         */
/*   n2 = rms_norm(x1, post_norm); out = x1 + MoE(n2).                        */
/* MoE weights as in orc_moe_forward (shared expert first when n_shared = 1). */
/* Optional outputs (NULL to skip): attn_out [T, d] (the attention sub-layer  */
/* output before the residual), x1 [T, d], moe_out [T, d].                    */
/* ------------------------------------------------------------------------ */
ORC_API int orc_block_forward(
    const float *x, size_t batch, size_t seq_len, size_t d, size_t Hq, size_t Hkv,
    size_t hd, const float *input_norm, const float *post_norm, float eps,
    const float *wq, const float *wk, const float *wv, const float *wo,
    const float *cos_cache, const float *sin_cache, size_t pos_offset, size_t f,
    size_t E, size_t k, size_t n_shared, const float *w_router,
    const float *router_bias, const float *const *w_gate,
    const float *const *w_up, const float *const *w_down, float *out,
    float *attn_out, float *x1_out, float *moe_out) {
  const size_t T = batch * seq_len;
  int rc = 0;
  float *n1 = (float *)malloc(sizeof(float) * T * d);
  float *att = attn_out ? attn_out : (float *)malloc(sizeof(float) * T * d);
  float *x1 = x1_out ? x1_out : (float *)malloc(sizeof(float) * T * d);
  float *mo = moe_out ? moe_out : (float *)malloc(sizeof(float) * T * d);
  if (!n1 || !att || !x1 || !mo) rc = -1;
  if (rc == 0) orc_rms_norm(x, input_norm, n1, T, d, eps);
  for (size_t b = 0; rc == 0 && b < batch; ++b)
    rc = orc_attention_forward(n1 + b * seq_len * d, seq_len, d, Hq, Hkv, hd, wq, wk, wv,
                               wo, cos_cache, sin_cache, pos_offset,
                               att + b * seq_len * d, NULL);
  if (rc == 0) {
    orc_add_tensors(x, att, x1, T * d);
    orc_rms_norm(x1, post_norm, n1, T, d, eps);
    rc = orc_moe_forward(n1, T, d, f, E, k, n_shared, w_router, router_bias, NULL, 0, w_gate,
                         w_up, w_down, mo, NULL, NULL, NULL, NULL, NULL, NULL, NULL);
  }
  if (rc == 0) orc_add_tensors(x1, mo, out, T * d);
  free(n1);
  if (!attn_out) free(att);
  if (!x1_out) free(x1);
  if (!moe_out) free(mo);
  return rc;
}

/* Number of OpenMP threads the oracle will use (1 without OpenMP). */
ORC_API int orc_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

ORC_API void orc_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}
