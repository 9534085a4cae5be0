// engine.hip -- the MoE layer engine: packed weights + workspace + forward.
//
// Replaces the MoE part of the reference's GpuModelEngine
// (crates/prichs-cuda/src/engine.rs:363-649 allocation, 668-689 upload,
// 1917-2239 forward) and the host routing of crates/prichs-model/src/
// model.rs:1125-1177.  All memory is allocated at creation for max_tokens;
// a forward is five launches on one stream with no host synchronisation:
//
//   router_topk -> permute -> grouped gate/up+SwiGLU -> grouped down -> combine
//
// Row space of act / y: routed rows (expert ascending, token ascending), then
// the shared expert's T rows (group E).
//
// Backward (after enable_backward): on the forward's stash, whose gate/up
// GEMM then also keeps the pre-activations,
//   rows pass (dY, gathered x, router scalars) -> dW_down -> dA = dY Wd^T
//   with the SwiGLU backward in its epilogue (bf16, tiled sizes; else two
//   launches) -> dX = [dG dU] [Wg Wu]^T -> combine (router VJP, d_x) ->
//   dW_gate / dW_up -> dW_router (two passes)
// with the transposed weights packed at upload.
#include <algorithm>
#include <cstring>
#include <new>
#include <vector>

#include "common.hpp"

struct prichs_moe_engine {
  int device = 0;
  size_t d = 0, f = 0, E = 0, k = 0, S = 0, max_tokens = 0;
  int dtype = PRICHS_DTYPE_BF16;
  bool uploaded = false;

  void *arena = nullptr;  // one allocation for weights + workspace
  float *w_router = nullptr;
  float *w_router_lds = nullptr;  // W^T [E][d + 4] for the router kernel's LDS (may be null)
  float *router_bias = nullptr;
  void *w_gate_up = nullptr;
  void *w_down = nullptr;
  float *logits = nullptr;
  int32_t *topk_idx = nullptr;
  float *topk_w = nullptr;
  int32_t *block_counts = nullptr;
  int32_t *offsets = nullptr;
  int32_t *row_token = nullptr;
  float *row_weight = nullptr;
  int32_t *token_row = nullptr;
  void *act = nullptr;
  void *y = nullptr;
  // Decode path (decode_gate_up_router / decode_down): the dense gate/up
  // activations [(E + 1) dense_tokens][f] and the dense row of every row.
  size_t dense_tokens = 0;
  void *act_dense = nullptr;
  int32_t *dense_row = nullptr;
  size_t gu_elems = 0, dn_elems = 0;  // packed elements per expert
  size_t last_T = 0;
  bool stash_valid = false;  // a forward's intermediates await a backward

  // Backward: a second allocation made by enable_backward.
  bool bwd = false;
  void *bwd_arena = nullptr;
  void *w_down_t = nullptr;  // per group packed [roundup(f, 256)][d]: B of dA = dY Wd^T
  void *w_cat = nullptr;     // per group packed [roundup(d, 256)][np_gu]: B of dX
  size_t np_gu = 0, dt_elems = 0, cat_elems = 0;
  void *gu = nullptr;        // [rows, np_gu] gate/up pre-activations, then dG / dU
  void *dy = nullptr;        // [rows, d] dY, then dX
  void *xg = nullptr;        // [rows, d] x gathered by row
  float *scal = nullptr;     // [rows] router scalars of the routed rows
  float *dlr = nullptr;      // [max_tokens * k] d_logit of each routed row
  float *wrt = nullptr;      // [E, d] router weights transposed
  float *rpart = nullptr;    // router weight-gradient partial sums
  float *wpart = nullptr;    // weight-gradient split-K partials

  // Stage timing: `slots` sets of PRICHS_NUM_STAGES events, filled in turn
  // by timed forwards (created by set_timing, never inside forward).
  int slots = 0;
  int recorded = 0;
  std::vector<hipEvent_t> ev;
  // The same for backwards: PRICHS_NUM_BWD_STAGES events per backward.
  int brecorded = 0;
  std::vector<hipEvent_t> bev;
};

namespace prichs {
namespace {

struct DeviceGuard {
  int prev = -1;
  bool ok = true;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) {
      ok = false;
      return;
    }
    if (prev != dev && hipSetDevice(dev) != hipSuccess) ok = false;
  }
  ~DeviceGuard() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

struct Carve {
  size_t off = 0;
  size_t take(size_t bytes) {
    const size_t at = off;
    off = roundup(off + bytes, 256);
    return at;
  }
};

}  // namespace
}  // namespace prichs

using namespace prichs;

extern "C" int prichs_moe_engine_create(size_t d, size_t f, size_t E, size_t k, size_t n_shared,
                                        int dtype, size_t max_tokens, prichs_moe_engine **out) {
  PRICHS_REQUIRE(out != nullptr, "engine_create: null output handle");
  *out = nullptr;
  PRICHS_REQUIRE(dtype_ok(dtype), "engine_create: bad dtype %d", dtype);
  PRICHS_REQUIRE(E >= 1 && E <= PRICHS_MAX_EXPERTS, "engine_create: E=%zu outside [1, %d]", E,
                 PRICHS_MAX_EXPERTS);
  PRICHS_REQUIRE(k >= 1 && k <= E && k <= PRICHS_MAX_TOPK,
                 "engine_create: k=%zu invalid for E=%zu", k, E);
  PRICHS_REQUIRE(n_shared <= 1, "engine_create: n_shared=%zu (0 or 1 supported)", n_shared);
  PRICHS_REQUIRE(max_tokens >= 1 && max_tokens <= (size_t)INT32_MAX / (k + 1),
                 "engine_create: max_tokens=%zu outside [1, %zu]", max_tokens,
                 (size_t)INT32_MAX / (k + 1));
  const size_t gu = prichs_packed_gate_up_elems(d, f, dtype);
  const size_t dn = prichs_packed_down_elems(d, f, dtype);
  {
    // Shape support is the grouped GEMMs' (multiples of their K tile).
    if (d == 0 || f == 0) return fail(PRICHS_ERR_UNSUPPORTED, "engine_create: d and f must be >0");
    const size_t q = dtype == PRICHS_DTYPE_BF16 ? 64 : 16;
    if (d % q || f % q)
      return fail(PRICHS_ERR_UNSUPPORTED,
                  "engine_create: d=%zu and f=%zu must be multiples of %zu for this dtype", d, f,
                  q);
  }
  const size_t es = dtype_size(dtype);
  const size_t G = E + n_shared;
  const size_t Tm = max_tokens;
  const size_t rows = Tm * k + n_shared * Tm;
  const size_t nb = prichs_router_num_blocks(Tm, E);

  prichs_moe_engine *eng = new (std::nothrow) prichs_moe_engine();
  if (!eng) return fail(PRICHS_ERR_CAPACITY, "engine_create: out of host memory");
  eng->d = d;
  eng->f = f;
  eng->E = E;
  eng->k = k;
  eng->S = n_shared;
  eng->dtype = dtype;
  eng->max_tokens = Tm;
  eng->gu_elems = gu;
  eng->dn_elems = dn;

  Carve c;
  const size_t o_router = c.take(sizeof(float) * d * E);
  const size_t n_rlds = router_lds_layout_elems(d, E);
  const size_t o_rlds = c.take(sizeof(float) * (n_rlds > 0 ? n_rlds : 1));
  const size_t o_bias = c.take(sizeof(float) * E);
  const size_t o_gu = c.take(es * gu * G);
  const size_t o_dn = c.take(es * dn * G);
  const size_t o_logits = c.take(sizeof(float) * Tm * E);
  const size_t o_idx = c.take(sizeof(int32_t) * Tm * k);
  const size_t o_w = c.take(sizeof(float) * Tm * k);
  const size_t o_bc = c.take(sizeof(int32_t) * nb * E);
  const size_t o_off = c.take(sizeof(int32_t) * (E + 2));
  const size_t o_rt = c.take(sizeof(int32_t) * (Tm * k + Tm));
  const size_t o_rw = c.take(sizeof(float) * Tm * k);
  const size_t o_tr = c.take(sizeof(int32_t) * Tm * k);
  const size_t o_act = c.take(es * rows * f);
  const size_t o_y = c.take(es * rows * d);
  // Decode buffers for batches one router workgroup covers (32 tokens).
  const size_t Td = (dtype == PRICHS_DTYPE_BF16 && n_shared == 1) ? std::min<size_t>(Tm, 32) : 0;
  const size_t o_actd = c.take(es * (E + 1) * Td * f + 1);
  const size_t o_drow = c.take(sizeof(int32_t) * (Td * k + Td) + 1);

  int rc = PRICHS_OK;
  if (hipGetDevice(&eng->device) != hipSuccess) {
    rc = fail(PRICHS_ERR_HIP, "engine_create: no HIP device");
  } else {
    hipError_t e = hipMalloc(&eng->arena, c.off);
    if (e != hipSuccess) {
      eng->arena = nullptr;
      rc = fail(PRICHS_ERR_CAPACITY, "engine_create: hipMalloc(%zu bytes): %s", c.off,
                hipGetErrorString(e));
    }
  }
  if (rc != PRICHS_OK) {
    prichs_moe_engine_destroy(eng);
    return rc;
  }
  char *base = static_cast<char *>(eng->arena);
  eng->w_router = reinterpret_cast<float *>(base + o_router);
  eng->w_router_lds = n_rlds > 0 ? reinterpret_cast<float *>(base + o_rlds) : nullptr;
  eng->router_bias = reinterpret_cast<float *>(base + o_bias);
  eng->w_gate_up = base + o_gu;
  eng->w_down = base + o_dn;
  eng->logits = reinterpret_cast<float *>(base + o_logits);
  eng->topk_idx = reinterpret_cast<int32_t *>(base + o_idx);
  eng->topk_w = reinterpret_cast<float *>(base + o_w);
  eng->block_counts = reinterpret_cast<int32_t *>(base + o_bc);
  eng->offsets = reinterpret_cast<int32_t *>(base + o_off);
  eng->row_token = reinterpret_cast<int32_t *>(base + o_rt);
  eng->row_weight = reinterpret_cast<float *>(base + o_rw);
  eng->token_row = reinterpret_cast<int32_t *>(base + o_tr);
  eng->act = base + o_act;
  eng->dense_tokens = Td;
  eng->act_dense = Td > 0 ? base + o_actd : nullptr;
  eng->dense_row = Td > 0 ? reinterpret_cast<int32_t *>(base + o_drow) : nullptr;
  eng->y = base + o_y;
  *out = eng;
  return PRICHS_OK;
}

extern "C" int prichs_moe_engine_destroy(prichs_moe_engine *eng) {
  if (!eng) return PRICHS_OK;
  int rc = PRICHS_OK;
  {
    DeviceGuard g(eng->device);
    for (hipEvent_t e : eng->ev)
      if (e) (void)hipEventDestroy(e);
    for (hipEvent_t e : eng->bev)
      if (e) (void)hipEventDestroy(e);
    if (eng->arena && hipFree(eng->arena) != hipSuccess)
      rc = fail(PRICHS_ERR_HIP, "engine_destroy: hipFree failed");
    if (eng->bwd_arena && hipFree(eng->bwd_arena) != hipSuccess)
      rc = fail(PRICHS_ERR_HIP, "engine_destroy: hipFree failed");
  }
  delete eng;
  return rc;
}

extern "C" int prichs_moe_engine_upload(prichs_moe_engine *eng, const float *w_router,
                                        const float *router_bias, const float *const *gate,
                                        const float *const *up, const float *const *down) {
  PRICHS_REQUIRE(eng != nullptr, "engine_upload: null engine");
  PRICHS_REQUIRE(w_router && gate && up && down, "engine_upload: null pointer argument");
  const size_t G = eng->E + eng->S;
  for (size_t i = 0; i < G; ++i)
    PRICHS_REQUIRE(gate[i] && up[i] && down[i], "engine_upload: null weight for expert slot %zu",
                   i);
  const size_t es = dtype_size(eng->dtype);
  std::vector<char> gu(es * eng->gu_elems * G), dn(es * eng->dn_elems * G);
  // Reference order is [shared, routed 0..E-1]; packed order is
  // [routed 0..E-1, shared] so the shared group follows the routed rows.
  for (size_t slot = 0; slot < G; ++slot) {
    const size_t grp = slot < eng->S ? eng->E : slot - eng->S;
    int rc = prichs_pack_gate_up(gate[slot], up[slot], eng->d, eng->f, eng->dtype,
                                 gu.data() + es * eng->gu_elems * grp);
    if (rc) return rc;
    rc = prichs_pack_down(down[slot], eng->d, eng->f, eng->dtype,
                          dn.data() + es * eng->dn_elems * grp);
    if (rc) return rc;
  }
  // Backward operands: B[n][k] = Wd[n][k] (n < f, k < d) for dA = dY Wd^T,
  // and B[n][p] = Wg[n][c] / Wu[n][c] for packed gate / up column p of
  // column c (zero on padding) for dX = [dG dU] [Wg Wu]^T.
  std::vector<char> dt, cat;
  if (eng->bwd) {
    const size_t d = eng->d, f = eng->f, np = eng->np_gu;
    dt.resize(es * eng->dt_elems * G);
    cat.resize(es * eng->cat_elems * G);
    std::vector<float> wt(d * f), wc(np * d);
    for (size_t slot = 0; slot < G; ++slot) {
      const size_t grp = slot < eng->S ? eng->E : slot - eng->S;
      for (size_t n = 0; n < f; ++n)
        for (size_t kk = 0; kk < d; ++kk) wt[kk * f + n] = down[slot][n * d + kk];
      int rc = prichs_pack_weight(wt.data(), d, f, eng->dtype, dt.data() + es * eng->dt_elems * grp);
      if (rc) return rc;
      const size_t il = prichs_gate_up_interleave(eng->dtype);
      for (size_t p = 0; p < np; ++p) {
        const size_t blk = p / (2 * il), w = p % (2 * il);
        const size_t c = blk * il + (w < il ? w : w - il);
        const float *src = w < il ? gate[slot] : up[slot];
        for (size_t n = 0; n < d; ++n) wc[p * d + n] = c < f ? src[n * f + c] : 0.0f;
      }
      rc = prichs_pack_weight(wc.data(), np, d, eng->dtype, cat.data() + es * eng->cat_elems * grp);
      if (rc) return rc;
    }
  }
  std::vector<float> bias(eng->E, 0.0f);
  if (router_bias) std::memcpy(bias.data(), router_bias, sizeof(float) * eng->E);
  DeviceGuard g(eng->device);
  if (!g.ok) return fail(PRICHS_ERR_HIP, "engine_upload: cannot select device %d", eng->device);
  PRICHS_HIP_TRY(hipMemcpy(eng->w_router, w_router, sizeof(float) * eng->d * eng->E,
                           hipMemcpyHostToDevice),
                 "engine_upload: router");
  if (eng->w_router_lds != nullptr) {
    std::vector<float> wl(router_lds_layout_elems(eng->d, eng->E));
    router_lds_layout(w_router, eng->d, eng->E, wl.data());
    PRICHS_HIP_TRY(hipMemcpy(eng->w_router_lds, wl.data(), sizeof(float) * wl.size(),
                             hipMemcpyHostToDevice),
                   "engine_upload: router (router layout)");
  }
  PRICHS_HIP_TRY(hipMemcpy(eng->router_bias, bias.data(), sizeof(float) * eng->E,
                           hipMemcpyHostToDevice),
                 "engine_upload: router bias");
  PRICHS_HIP_TRY(hipMemcpy(eng->w_gate_up, gu.data(), gu.size(), hipMemcpyHostToDevice),
                 "engine_upload: gate/up");
  PRICHS_HIP_TRY(hipMemcpy(eng->w_down, dn.data(), dn.size(), hipMemcpyHostToDevice),
                 "engine_upload: down");
  if (eng->bwd) {
    std::vector<float> wrt(eng->E * eng->d);
    for (size_t e = 0; e < eng->E; ++e)
      for (size_t c = 0; c < eng->d; ++c) wrt[e * eng->d + c] = w_router[c * eng->E + e];
    PRICHS_HIP_TRY(hipMemcpy(eng->wrt, wrt.data(), sizeof(float) * wrt.size(),
                             hipMemcpyHostToDevice),
                   "engine_upload: transposed router");
    PRICHS_HIP_TRY(hipMemcpy(eng->w_down_t, dt.data(), dt.size(), hipMemcpyHostToDevice),
                   "engine_upload: transposed down");
    PRICHS_HIP_TRY(hipMemcpy(eng->w_cat, cat.data(), cat.size(), hipMemcpyHostToDevice),
                   "engine_upload: transposed gate/up");
  }
  eng->stash_valid = false;
  PRICHS_HIP_TRY(hipDeviceSynchronize(), "engine_upload: synchronize");
  eng->uploaded = true;
  return PRICHS_OK;
}

// Block `layer` of a reference weight file (model.rs:312-338) into the
// engine: lengths are checked against the engine's d, f, E before anything
// is uploaded.
extern "C" int prichs_moe_engine_upload_checkpoint(prichs_moe_engine *eng,
                                                   const prichs_checkpoint *ck, size_t layer,
                                                   const float *router_bias) {
  PRICHS_REQUIRE(eng != nullptr && ck != nullptr, "engine_upload_checkpoint: null pointer argument");
  if (eng->S != 1)
    return fail(PRICHS_ERR_UNSUPPORTED,
                "engine_upload_checkpoint: a checkpoint layer has one shared expert (moe.rs:61), "
                "the engine has n_shared=%zu",
                eng->S);
  CheckpointMoe w;
  if (int rc = checkpoint_moe_weights(ck, layer, eng->d, eng->f, eng->E, w)) return rc;
  return prichs_moe_engine_upload(eng, w.router.data(), router_bias, w.pg.data(), w.pu.data(),
                                  w.pd.data());
}

extern "C" int prichs_moe_engine_set_router_bias(prichs_moe_engine *eng, const float *router_bias) {
  PRICHS_REQUIRE(eng && router_bias, "engine_set_router_bias: null pointer argument");
  DeviceGuard g(eng->device);
  if (!g.ok) return fail(PRICHS_ERR_HIP, "engine_set_router_bias: cannot select device");
  PRICHS_HIP_TRY(hipMemcpy(eng->router_bias, router_bias, sizeof(float) * eng->E,
                           hipMemcpyHostToDevice),
                 "engine_set_router_bias");
  return PRICHS_OK;
}

namespace prichs {
namespace {
// MoELayer::update_aux_free_bias (crates/prichs-model/src/moe.rs:228-245) with
// the counts of its call site (model.rs:1541-1547: assignments per expert over
// the last batch, = offsets[e+1] - offsets[e]) and total_tokens = T.  f32
// arithmetic in the reference's order: target = k / E, actual = count / T,
// diff = target - actual, bias += gamma * diff (division correctly rounded,
// no contraction).
__global__ void aux_free_bias_kernel(float *bias, const int32_t *offsets, int E, int T, int k,
                                     float gamma) {
#pragma clang fp contract(off)
  const int i = threadIdx.x;
  if (i >= E) return;
  const float target = (float)k / (float)E;
  const float actual = (float)(offsets[i + 1] - offsets[i]) / (float)T;
  const float diff = target - actual;
  const float step = gamma * diff;
  bias[i] = bias[i] + step;
}
}  // namespace
}  // namespace prichs

extern "C" int prichs_moe_engine_update_router_bias(prichs_moe_engine *eng, float gamma,
                                                    void *stream) {
  PRICHS_REQUIRE(eng != nullptr, "engine_update_router_bias: null engine");
  if (!eng->uploaded) return fail(PRICHS_ERR_STATE, "engine_update_router_bias: weights not uploaded");
  if (eng->last_T == 0) return PRICHS_OK;  // the reference returns on total_tokens == 0
  DeviceGuard g(eng->device);
  if (!g.ok) return fail(PRICHS_ERR_HIP, "engine_update_router_bias: cannot select device");
  hipLaunchKernelGGL(aux_free_bias_kernel, dim3(1), dim3(PRICHS_MAX_EXPERTS), 0, as_stream(stream),
                     eng->router_bias, eng->offsets, (int)eng->E, (int)eng->last_T, (int)eng->k,
                     gamma);
  PRICHS_LAUNCH_CHECK("engine_update_router_bias");
  return PRICHS_OK;
}

extern "C" int prichs_moe_engine_get_router_bias(const prichs_moe_engine *eng, float *out) {
  PRICHS_REQUIRE(eng && out, "engine_get_router_bias: null pointer argument");
  DeviceGuard g(eng->device);
  if (!g.ok) return fail(PRICHS_ERR_HIP, "engine_get_router_bias: cannot select device");
  PRICHS_HIP_TRY(hipMemcpy(out, eng->router_bias, sizeof(float) * eng->E, hipMemcpyDeviceToHost),
                 "engine_get_router_bias");
  return PRICHS_OK;
}

static int moe_finish(prichs_moe_engine *eng, size_t T, void *out, int out_dtype, void *stream,
                      const float *residual, void *moe_out, bool tm, hipEvent_t *ev);

// The forward; with residual != nullptr the combine writes the layer output
// to moe_out (bf16) and residual + that output to out (the block's final
// residual add, in the same kernel).
static int moe_forward_impl(prichs_moe_engine *eng, const void *x, size_t T,
                            const float *concept_bias, size_t n_concept, void *out, int out_dtype,
                            void *stream, const float *residual, void *moe_out) {
  PRICHS_REQUIRE(eng != nullptr, "engine_forward: null engine");
  PRICHS_REQUIRE(dtype_ok(out_dtype), "engine_forward: bad out dtype %d", out_dtype);
  if (!eng->uploaded) return fail(PRICHS_ERR_STATE, "engine_forward: weights not uploaded");
  if (T > eng->max_tokens)
    return fail(PRICHS_ERR_CAPACITY, "engine_forward: T=%zu exceeds max_tokens=%zu", T,
                eng->max_tokens);
  eng->stash_valid = false;
  if (T == 0) {
    eng->last_T = 0;
    eng->stash_valid = true;
    return PRICHS_OK;
  }
  PRICHS_REQUIRE(x && out, "engine_forward: null pointer argument");
  PRICHS_REQUIRE(concept_bias != nullptr || n_concept == 0,
                 "engine_forward: concept_bias is NULL but n_concept=%zu", n_concept);
  DeviceGuard g(eng->device);
  if (!g.ok) return fail(PRICHS_ERR_HIP, "engine_forward: cannot select device");
  hipStream_t s = as_stream(stream);
  const bool tm = eng->slots > 0 && eng->recorded < eng->slots;
  hipEvent_t *ev = tm ? &eng->ev[(size_t)eng->recorded * PRICHS_NUM_STAGES] : nullptr;
  const size_t G = eng->E + eng->S;
  const size_t rows = T * eng->k + eng->S * T;
  int rc;
  if (tm) PRICHS_HIP_TRY(hipEventRecord(ev[0], s), "engine_forward: event");
  if (!eng->bwd && T <= eng->dense_tokens &&
      decode_dense_applies(T, eng->d, eng->f, eng->E, eng->k, eng->S, eng->dtype, x,
                           eng->w_router)) {
    // Decode: the router (and the permutation) runs in the first workgroup
    // of the gate/up launch, which covers every token of every expert; the
    // down GEMM gathers the routed rows.  Events [0]-[2] bracket no work.
    if (tm) PRICHS_HIP_TRY(hipEventRecord(ev[1], s), "engine_forward: event");
    if (tm) PRICHS_HIP_TRY(hipEventRecord(ev[2], s), "engine_forward: event");
    rc = decode_gate_up_router(x, T, eng->d, eng->f, eng->E, eng->k, eng->w_router,
                               eng->w_router_lds, eng->router_bias, concept_bias, n_concept,
                               eng->logits, eng->topk_idx, eng->topk_w, eng->block_counts,
                               eng->offsets, eng->row_token, eng->row_weight, eng->token_row,
                               eng->dense_row, eng->w_gate_up, eng->act_dense, stream);
    if (rc) return rc;
    if (tm) PRICHS_HIP_TRY(hipEventRecord(ev[3], s), "engine_forward: event");
    rc = decode_down(eng->act_dense, eng->dense_row, eng->offsets, T, eng->d, eng->f, eng->E,
                     eng->k, eng->w_down, eng->y, eng->act, stream);
    if (rc) return rc;
    if (tm) PRICHS_HIP_TRY(hipEventRecord(ev[4], s), "engine_forward: event");
    return moe_finish(eng, T, out, out_dtype, stream, residual, moe_out, tm, ev);
  }
  if (prichs_router_num_blocks(T, eng->E) == 1) {
    // Decode-sized batch: the router's one workgroup also writes the
    // permutation (the permute stage then times as zero).
    rc = router_topk_permute(x, eng->dtype, eng->w_router, eng->router_bias, concept_bias,
                             n_concept, T, eng->d, eng->E, eng->k, eng->logits, eng->topk_idx,
                             eng->topk_w, eng->block_counts, eng->offsets, eng->row_token,
                             eng->row_weight, eng->token_row, stream, eng->w_router_lds);
    if (rc) return rc;
    if (tm) PRICHS_HIP_TRY(hipEventRecord(ev[1], s), "engine_forward: event");
  } else {
    rc = router_topk_lds(x, eng->dtype, eng->w_router, eng->w_router_lds, eng->router_bias,
                         concept_bias, n_concept, T, eng->d, eng->E, eng->k, eng->logits,
                         eng->topk_idx, eng->topk_w, eng->block_counts, stream);
    if (rc) return rc;
    if (tm) PRICHS_HIP_TRY(hipEventRecord(ev[1], s), "engine_forward: event");
    rc = prichs_permute(eng->topk_idx, eng->topk_w, eng->block_counts, T, eng->E, eng->k,
                        eng->offsets, eng->row_token, eng->row_weight, eng->token_row, stream);
    if (rc) return rc;
  }
  if (tm) PRICHS_HIP_TRY(hipEventRecord(ev[2], s), "engine_forward: event");
  // No group holds more than T rows (a token picks an expert at most once).
  // With the backward enabled the GEMM also keeps the gate/up pre-activations.
  rc = grouped_gate_up_swiglu_rows(x, eng->row_token, eng->offsets, G, rows, T, eng->w_gate_up,
                                   eng->d, eng->f, eng->dtype, eng->act, stream,
                                   eng->bwd ? eng->gu : nullptr);
  if (rc) return rc;
  if (tm) PRICHS_HIP_TRY(hipEventRecord(ev[3], s), "engine_forward: event");
  rc = grouped_down_rows(eng->act, eng->offsets, G, rows, T, eng->w_down, eng->d, eng->f,
                         eng->dtype, eng->y, stream);
  if (rc) return rc;
  if (tm) PRICHS_HIP_TRY(hipEventRecord(ev[4], s), "engine_forward: event");
  return moe_finish(eng, T, out, out_dtype, stream, residual, moe_out, tm, ev);
}

// The combine (with the block's residual add when residual is set) and the
// forward's bookkeeping.
static int moe_finish(prichs_moe_engine *eng, size_t T, void *out, int out_dtype, void *stream,
                      const float *residual, void *moe_out, bool tm, hipEvent_t *ev) {
  hipStream_t s = as_stream(stream);
  // Without the backward nothing reads y after the combine, so the combine
  // streams it (non-temporal loads): the 75 MB of y at config 2 then no longer
  // push the layer's weights out of the memory-side cache between forwards
  // (repeated config-2 forwards: 2-11 us less per layer by box, although the
  // combine itself takes 2 us more; with flushed caches 3 us more).  With the
  // backward enabled the rows pass reads y again, and streaming it cost 2 us
  // per training step.
  const bool y_last_use = !eng->bwd;
  int rc;
  if (residual != nullptr && eng->dtype == PRICHS_DTYPE_BF16) {
    rc = moe_combine_residual(eng->y, eng->topk_idx, eng->topk_w, eng->token_row, T, eng->d,
                              eng->k, (int)eng->S, moe_out, residual, out, out_dtype, stream,
                              y_last_use);
  } else if (residual != nullptr) {
    rc = moe_combine(eng->y, eng->dtype, eng->topk_idx, eng->topk_w, eng->token_row, T, eng->d,
                     eng->k, (int)eng->S, moe_out, PRICHS_DTYPE_BF16, stream, y_last_use);
    if (!rc)
      rc = prichs_add(residual, PRICHS_DTYPE_F32, moe_out, PRICHS_DTYPE_BF16, out, out_dtype,
                      T * eng->d, stream);
  } else {
    rc = moe_combine(eng->y, eng->dtype, eng->topk_idx, eng->topk_w, eng->token_row, T, eng->d,
                     eng->k, (int)eng->S, out, out_dtype, stream, y_last_use);
  }
  if (rc) return rc;
  if (tm) PRICHS_HIP_TRY(hipEventRecord(ev[5], s), "engine_forward: event");
  if (tm) ++eng->recorded;
  eng->last_T = T;
  eng->stash_valid = true;
  return PRICHS_OK;
}

extern "C" int prichs_moe_engine_forward(prichs_moe_engine *eng, const void *x, size_t T,
                                         const float *concept_bias, size_t n_concept, void *out,
                                         int out_dtype, void *stream) {
  return moe_forward_impl(eng, x, T, concept_bias, n_concept, out, out_dtype, stream, nullptr,
                          nullptr);
}

namespace prichs {
int moe_engine_forward_residual(prichs_moe_engine *eng, const void *x, size_t T,
                                const float *concept_bias, size_t n_concept, void *moe_out,
                                const float *residual, void *out, int out_dtype, void *stream) {
  PRICHS_REQUIRE(residual != nullptr && moe_out != nullptr,
                 "engine_forward_residual: null residual or moe_out");
  return moe_forward_impl(eng, x, T, concept_bias, n_concept, out, out_dtype, stream, residual,
                          moe_out);
}
}  // namespace prichs

extern "C" int prichs_moe_engine_enable_backward(prichs_moe_engine *eng) {
  PRICHS_REQUIRE(eng != nullptr, "engine_enable_backward: null engine");
  if (eng->bwd) return PRICHS_OK;
  if (eng->uploaded)
    return fail(PRICHS_ERR_STATE,
                "engine_enable_backward: call before upload (the upload packs the transposed "
                "weights)");
  if (eng->S != 1)
    return fail(PRICHS_ERR_UNSUPPORTED,
                "engine_enable_backward: the backward has one shared expert (moe.rs:61), the "
                "engine has n_shared=%zu",
                eng->S);
  const size_t d = eng->d, f = eng->f, E = eng->E, G = E + 1, Tm = eng->max_tokens;
  const size_t es = dtype_size(eng->dtype);
  const size_t rows = Tm * (eng->k + 1);
  const size_t np = prichs_packed_gate_up_elems(1, f, eng->dtype);  // packed rows of one K column
  // The bf16 weight-gradient kernel addresses its operands with 32-bit offsets.
  if (eng->dtype == PRICHS_DTYPE_BF16 && rows * std::max(np, d) * es >= (size_t)1 << 31)
    return fail(PRICHS_ERR_UNSUPPORTED,
                "engine_enable_backward: max_tokens=%zu makes operands of 2 GiB or more", Tm);
  eng->np_gu = np;
  eng->dt_elems = prichs_packed_weight_elems(d, f, eng->dtype);
  eng->cat_elems = prichs_packed_weight_elems(np, d, eng->dtype);
  Carve c;
  const size_t o_dt = c.take(es * eng->dt_elems * G);
  const size_t o_cat = c.take(es * eng->cat_elems * G);
  const size_t o_gu = c.take(es * rows * np);
  const size_t o_dy = c.take(es * rows * d);
  const size_t o_xg = c.take(es * rows * d);
  const size_t o_scal = c.take(sizeof(float) * rows);
  const size_t o_dl = c.take(sizeof(float) * Tm * eng->k);
  const size_t o_wrt = c.take(sizeof(float) * E * d);
  const size_t o_rp = c.take(sizeof(float) * bwd_router_part_elems(Tm, eng->k, d, E));
  const size_t o_wp =
      c.take(sizeof(float) * std::max(bwd_wgrad_part_elems(rows, d, np), bwd_wgrad_part_elems(rows, f, d)));
  DeviceGuard g(eng->device);
  if (!g.ok) return fail(PRICHS_ERR_HIP, "engine_enable_backward: cannot select device");
  hipError_t e = hipMalloc(&eng->bwd_arena, c.off);
  if (e != hipSuccess) {
    eng->bwd_arena = nullptr;
    return fail(PRICHS_ERR_CAPACITY, "engine_enable_backward: hipMalloc(%zu bytes): %s", c.off,
                hipGetErrorString(e));
  }
  char *base = static_cast<char *>(eng->bwd_arena);
  eng->w_down_t = base + o_dt;
  eng->w_cat = base + o_cat;
  eng->gu = base + o_gu;
  eng->dy = base + o_dy;
  eng->xg = base + o_xg;
  eng->scal = reinterpret_cast<float *>(base + o_scal);
  eng->dlr = reinterpret_cast<float *>(base + o_dl);
  eng->wrt = reinterpret_cast<float *>(base + o_wrt);
  eng->rpart = reinterpret_cast<float *>(base + o_rp);
  eng->wpart = reinterpret_cast<float *>(base + o_wp);
  eng->bwd = true;
  return PRICHS_OK;
}

namespace {
bool aligned16(const void *p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }
}  // namespace

extern "C" int prichs_moe_engine_backward(prichs_moe_engine *eng, const void *x,
                                          const void *d_out, size_t T, void *d_x, int d_x_dtype,
                                          const prichs_moe_grads *grads, int dx_weighting,
                                          void *stream) {
  PRICHS_REQUIRE(eng != nullptr && grads != nullptr, "engine_backward: null pointer argument");
  PRICHS_REQUIRE(dtype_ok(d_x_dtype), "engine_backward: bad d_x dtype %d", d_x_dtype);
  PRICHS_REQUIRE(dx_weighting == 1 || dx_weighting == 2,
                 "engine_backward: dx_weighting=%d (1 = chain rule, 2 = the reference's)",
                 dx_weighting);
  if (!eng->bwd)
    return fail(PRICHS_ERR_STATE, "engine_backward: enable_backward was not called before upload");
  if (!eng->uploaded) return fail(PRICHS_ERR_STATE, "engine_backward: weights not uploaded");
  if (!eng->stash_valid || eng->last_T != T)
    return fail(PRICHS_ERR_STATE,
                "engine_backward: needs the forward of this batch (T=%zu) right before it", T);
  const size_t d = eng->d, f = eng->f, E = eng->E, k = eng->k, G = E + 1;
  PRICHS_REQUIRE(grads->d_router && grads->d_gate && grads->d_up && grads->d_down,
                 "engine_backward: null gradient buffer");
  PRICHS_REQUIRE(grads->slot_stride >= d * f && grads->slot_stride % 4 == 0,
                 "engine_backward: slot_stride=%zu (a multiple of 4, at least d*f=%zu)",
                 grads->slot_stride, d * f);
  PRICHS_REQUIRE(aligned16(grads->d_router) && aligned16(grads->d_gate) &&
                     aligned16(grads->d_up) && aligned16(grads->d_down),
                 "engine_backward: gradient buffers must be 16-byte aligned");
  PRICHS_REQUIRE(grads->beta == 0 || grads->beta == 1,
                 "engine_backward: beta=%d (1 = add to the gradients, 0 = overwrite them)",
                 grads->beta);
  if (T == 0) {
    eng->stash_valid = false;
    if (grads->beta != 0) return PRICHS_OK;
    DeviceGuard g(eng->device);
    if (!g.ok) return fail(PRICHS_ERR_HIP, "engine_backward: cannot select device");
    return bwd_zero_grads(grads->d_router, d * E, grads->d_gate, grads->d_up, grads->d_down,
                          grads->slot_stride, G, d * f, as_stream(stream));
  }
  PRICHS_REQUIRE(x && d_out && d_x, "engine_backward: null pointer argument");
  PRICHS_REQUIRE(aligned16(x) && aligned16(d_out) && aligned16(d_x),
                 "engine_backward: x, d_out and d_x must be 16-byte aligned");
  DeviceGuard g(eng->device);
  if (!g.ok) return fail(PRICHS_ERR_HIP, "engine_backward: cannot select device");
  eng->stash_valid = false;
  hipStream_t s = as_stream(stream);
  const int dt = eng->dtype;
  const size_t rows = T * (k + 1), routed = T * k, np = eng->np_gu;
  const size_t np_f = roundup(f, 256), np_d = roundup(d, 256);
  const bool tm = eng->slots > 0 && eng->brecorded < eng->slots;
  hipEvent_t *ev = tm ? &eng->bev[(size_t)eng->brecorded * PRICHS_NUM_BWD_STAGES] : nullptr;
  int rc;
#define PRICHS_BWD_MARK(i) \
  if (tm) PRICHS_HIP_TRY(hipEventRecord(ev[i], s), "engine_backward: event")
  PRICHS_BWD_MARK(0);
  // (Stage 0, the gate/up pre-activations, is written by the forward's
  // gate/up GEMM when the backward is enabled; its interval stays empty.)
  // The shared expert's rows of dY and xg are d_out and x themselves (weight
  // 1, rows in token order).  Where the bf16 tiled kernels run (the fused dA
  // + SwiGLU backward applies), dW_down, dA and dW_gate/up read those rows
  // from d_out and x directly and the rows pass covers the routed rows only.
  // (dW_gate/up reads x after the combine has written d_x, so not when d_x
  // shares memory with x; d_out is read before the combine.)
  const uintptr_t x0 = reinterpret_cast<uintptr_t>(x), dx0 = reinterpret_cast<uintptr_t>(d_x);
  const bool dx_overlaps_x =
      dx0 < x0 + T * d * dtype_size(dt) && x0 < dx0 + T * d * dtype_size(d_x_dtype);
  const bool lean = eng->S == 1 && !dx_overlaps_x &&
                    dact_swiglu_bwd_fusable(d, np_f, eng->gu, np, f, rows, T, dt);
  WgradAlt alt_dy, alt_x;
  if (lean) {
    alt_dy.B = d_out;
    alt_x.A = x;
    alt_dy.g = alt_x.g = E;
    alt_dy.row0 = alt_x.row0 = routed;
    alt_dy.rows = alt_x.rows = T;
  }
  PRICHS_BWD_MARK(1);
  rc = bwd_rows(x, d_out, eng->y, eng->token_row, eng->row_weight, T, k, !lean, d, dt, eng->dy,
                eng->xg, eng->scal, s);
  if (rc) return rc;
  PRICHS_BWD_MARK(2);
  rc = bwd_wgrad(false, eng->act, f, eng->dy, d, rows, eng->offsets, G, E, f, d, grads->d_down,
                 nullptr, d, grads->slot_stride, f, dt, eng->wpart, grads->beta, s, alt_dy);
  if (rc) return rc;
  PRICHS_BWD_MARK(3);
  // dA = dY Wd^T with the SwiGLU backward in its epilogue (dG, dU into gu in
  // place; the SwiGLU interval then stays empty), or dA into act and the
  // separate SwiGLU backward where the fused kernel does not apply.
  bool fused = false;
  rc = grouped_dact_swiglu_bwd(eng->dy, d, eng->w_down_t, eng->dt_elems, np_f, eng->gu, np, f,
                               eng->offsets, G, rows, T, dt, stream, &fused,
                               lean ? d_out : nullptr, E, routed);
  if (rc) return rc;
  if (lean && !fused)
    return fail(PRICHS_ERR_STATE, "engine_backward: the dA launch did not take the shared rows");
  if (!fused) {
    rc = grouped_gemm_rows(eng->dy, nullptr, d, eng->w_down_t, eng->dt_elems, np_f, d, eng->act,
                           f, f, eng->offsets, G, rows, T, dt, stream);
    if (rc) return rc;
  }
  PRICHS_BWD_MARK(4);
  if (!fused) {
    rc = bwd_swiglu(eng->gu, eng->act, rows, f, np, dt, s);
    if (rc) return rc;
  }
  // dX, then the combine that reads it, then the weight gradients: each
  // reads what the launch before it wrote while that is still in the memory-
  // side cache (dX after dG/dU: 8 us faster than after dW_gate/up's partials
  // and output; dW_router after dW_gate/up, which reads the same gathered x).
  PRICHS_BWD_MARK(5);
  rc = grouped_gemm_rows(eng->gu, nullptr, np, eng->w_cat, eng->cat_elems, np_d, np, eng->dy, d, d,
                         eng->offsets, G, rows, T, dt, stream);
  if (rc) return rc;
  PRICHS_BWD_MARK(6);
  rc = bwd_combine(eng->dy, eng->scal, eng->topk_idx, eng->topk_w, eng->token_row, eng->wrt, T, d,
                   k, dx_weighting, dt, eng->dlr, d_x, d_x_dtype, s);
  if (rc) return rc;
  PRICHS_BWD_MARK(7);
  rc = bwd_wgrad(true, eng->xg, d, eng->gu, np, rows, eng->offsets, G, E, d, np, grads->d_gate,
                 grads->d_up, f, grads->slot_stride, f, dt, eng->wpart, grads->beta, s, alt_x);
  if (rc) return rc;
  PRICHS_BWD_MARK(8);
  rc = bwd_router_wgrad(eng->xg, eng->dlr, eng->offsets, T, k, d, E, dt, eng->rpart,
                        grads->d_router, grads->beta, s);
  if (rc) return rc;
  PRICHS_BWD_MARK(9);
#undef PRICHS_BWD_MARK
  if (tm) ++eng->brecorded;
  return PRICHS_OK;
}

extern "C" int prichs_moe_engine_stash(const prichs_moe_engine *eng, prichs_moe_stash *out) {
  PRICHS_REQUIRE(eng && out, "engine_stash: null pointer argument");
  out->T = eng->last_T;
  out->router_logits = eng->logits;
  out->selected_experts = eng->topk_idx;
  out->gating_weights = eng->topk_w;
  out->offsets = eng->offsets;
  out->row_token = eng->row_token;
  out->row_weight = eng->row_weight;
  out->token_row = eng->token_row;
  out->act = eng->act;
  out->y = eng->y;
  return PRICHS_OK;
}

extern "C" int prichs_moe_engine_set_timing(prichs_moe_engine *eng, int max_forwards) {
  PRICHS_REQUIRE(eng != nullptr, "engine_set_timing: null engine");
  PRICHS_REQUIRE(max_forwards >= 0 && max_forwards <= 1 << 16,
                 "engine_set_timing: max_forwards=%d outside [0, 65536]", max_forwards);
  DeviceGuard g(eng->device);
  if (!g.ok) return fail(PRICHS_ERR_HIP, "engine_set_timing: cannot select device");
  const size_t need = (size_t)max_forwards * PRICHS_NUM_STAGES;
  while (eng->ev.size() < need) {
    hipEvent_t e = nullptr;
    PRICHS_HIP_TRY(hipEventCreate(&e), "engine_set_timing: hipEventCreate");
    eng->ev.push_back(e);
  }
  const size_t bneed = eng->bwd ? (size_t)max_forwards * PRICHS_NUM_BWD_STAGES : 0;
  while (eng->bev.size() < bneed) {
    hipEvent_t e = nullptr;
    PRICHS_HIP_TRY(hipEventCreate(&e), "engine_set_timing: hipEventCreate");
    eng->bev.push_back(e);
  }
  eng->slots = max_forwards;
  eng->recorded = 0;
  eng->brecorded = 0;
  return PRICHS_OK;
}

extern "C" int prichs_moe_engine_stage_ms(prichs_moe_engine *eng, float *ms_out,
                                          int *n_forwards) {
  PRICHS_REQUIRE(eng && ms_out, "engine_stage_ms: null pointer argument");
  if (eng->recorded == 0)
    return fail(PRICHS_ERR_STATE, "engine_stage_ms: no timed forward since set_timing");
  DeviceGuard g(eng->device);
  double acc[PRICHS_NUM_STAGES] = {0};
  for (int f = 0; f < eng->recorded; ++f) {
    hipEvent_t *ev = &eng->ev[(size_t)f * PRICHS_NUM_STAGES];
    PRICHS_HIP_TRY(hipEventSynchronize(ev[PRICHS_NUM_STAGES - 1]), "engine_stage_ms: sync");
    float ms = 0.f;
    for (int i = 0; i + 1 < PRICHS_NUM_STAGES; ++i) {
      PRICHS_HIP_TRY(hipEventElapsedTime(&ms, ev[i], ev[i + 1]), "engine_stage_ms: elapsed");
      acc[i] += ms;
    }
    PRICHS_HIP_TRY(hipEventElapsedTime(&ms, ev[0], ev[PRICHS_NUM_STAGES - 1]),
                   "engine_stage_ms: elapsed");
    acc[PRICHS_NUM_STAGES - 1] += ms;
  }
  for (int i = 0; i < PRICHS_NUM_STAGES; ++i) ms_out[i] = (float)(acc[i] / eng->recorded);
  if (n_forwards) *n_forwards = eng->recorded;
  eng->recorded = 0;
  return PRICHS_OK;
}

extern "C" int prichs_moe_engine_backward_stage_ms(prichs_moe_engine *eng, float *ms_out,
                                                   int *n_backwards) {
  PRICHS_REQUIRE(eng && ms_out, "engine_backward_stage_ms: null pointer argument");
  if (eng->brecorded == 0)
    return fail(PRICHS_ERR_STATE, "engine_backward_stage_ms: no timed backward since set_timing");
  DeviceGuard g(eng->device);
  constexpr int N = PRICHS_NUM_BWD_STAGES;
  double acc[N] = {0};
  for (int b = 0; b < eng->brecorded; ++b) {
    hipEvent_t *ev = &eng->bev[(size_t)b * N];
    PRICHS_HIP_TRY(hipEventSynchronize(ev[N - 1]), "engine_backward_stage_ms: sync");
    float ms = 0.f;
    for (int i = 0; i + 1 < N; ++i) {
      PRICHS_HIP_TRY(hipEventElapsedTime(&ms, ev[i], ev[i + 1]), "engine_backward_stage_ms: elapsed");
      acc[i] += ms;
    }
    PRICHS_HIP_TRY(hipEventElapsedTime(&ms, ev[0], ev[N - 1]), "engine_backward_stage_ms: elapsed");
    acc[N - 1] += ms;
  }
  for (int i = 0; i < N; ++i) ms_out[i] = (float)(acc[i] / eng->brecorded);
  if (n_backwards) *n_backwards = eng->brecorded;
  eng->brecorded = 0;
  return PRICHS_OK;
}
