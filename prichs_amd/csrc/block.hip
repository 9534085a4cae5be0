// block.hip -- the PrichsBlock forward engine (config 5 caller of the MoE
// hot path).
//
// Restates crates/prichs-model/src/block.rs:50-68 on device for `batch`
// independent sequences of seq_len rows:
//   n1 = rms_norm(x, input_norm)                    prichs_rmsnorm_forward
//   qkv = n1 [Wq | Wk | Wv]                         prichs_gemm (one fused GEMM)
//   RoPE on the k columns of qkv in place           prichs_rope_forward_ld (one launch)
//   attn = causal GQA attention(RoPE(q), k, v)      attention kernel, rotating q on load
//   x1 = x + attn Wo                                prichs_gemm, then one kernel for the
//   n2 = rms_norm(x1, post_attn_norm)               residual add (x1 in f32) and the norm
//   out = x1 + MoE(n2)                              the MoE engine forward, whose combine
//                                                   also adds x1
// Everything is allocated at creation; a forward is a fixed sequence of
// launches on one stream with no host synchronisation.
#include <cstring>
#include <new>
#include <vector>

#include "common.hpp"

struct prichs_block_engine {
  int device = 0;
  size_t d = 0, Hq = 0, Hkv = 0, hd = 0, f = 0, E = 0, k = 0, S = 0, max_tokens = 0;
  size_t cache_rows = 0;
  float theta = 0.f, eps = 0.f;
  bool uploaded = false;
  size_t qkv_n = 0;  // columns of the fused projection: d + 2 * Hkv * hd
  size_t last_T = 0;

  void *arena = nullptr;
  void *w_qkv = nullptr;  // packed [roundup(qkv_n, 256)][d] bf16
  void *w_o = nullptr;    // packed [roundup(d, 256)][d] bf16
  float *input_norm = nullptr, *post_norm = nullptr;
  float *rope_cos = nullptr, *rope_sin = nullptr;
  void *n1 = nullptr, *qkv = nullptr, *attn = nullptr, *attn_out = nullptr;
  float *x1 = nullptr;
  void *n2 = nullptr, *moe_out = nullptr;
  prichs_moe_engine *moe = nullptr;
};

namespace prichs {
namespace {
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

extern "C" int prichs_block_engine_create(size_t d, size_t n_heads, size_t n_kv_heads, size_t f,
                                          size_t E, size_t k, size_t n_shared,
                                          size_t max_tokens, size_t max_seq_len,
                                          float rope_theta, float eps,
                                          prichs_block_engine **out) {
  PRICHS_REQUIRE(out != nullptr, "block_create: null output handle");
  *out = nullptr;
  PRICHS_REQUIRE(n_heads >= 1 && n_kv_heads >= 1 && n_heads % n_kv_heads == 0 && d % n_heads == 0,
                 "block_create: d=%zu, n_heads=%zu, n_kv_heads=%zu are inconsistent", d, n_heads,
                 n_kv_heads);
  if (d / n_heads != 128)
    return fail(PRICHS_ERR_UNSUPPORTED, "block_create: head_dim=%zu (the attention kernel needs 128)",
                d / n_heads);
  if (d % 64 || f % 64)
    return fail(PRICHS_ERR_UNSUPPORTED, "block_create: d=%zu and f=%zu must be multiples of 64", d, f);
  PRICHS_REQUIRE(max_tokens >= 1 && max_seq_len >= 1 && max_tokens * (d + 2 * d) <= (size_t)UINT32_MAX,
                 "block_create: max_tokens=%zu too large", max_tokens);
  PRICHS_REQUIRE(max_seq_len <= ((size_t)1 << 24), "block_create: max_seq_len too large");

  prichs_block_engine *eng = new (std::nothrow) prichs_block_engine();
  if (!eng) return fail(PRICHS_ERR_CAPACITY, "block_create: out of host memory");
  eng->d = d;
  eng->Hq = n_heads;
  eng->Hkv = n_kv_heads;
  eng->hd = d / n_heads;
  eng->f = f;
  eng->E = E;
  eng->k = k;
  eng->S = n_shared;
  eng->max_tokens = max_tokens;
  eng->cache_rows = max_seq_len;
  eng->theta = rope_theta;
  eng->eps = eps;
  eng->qkv_n = d + 2 * n_kv_heads * eng->hd;

  int rc = prichs_moe_engine_create(d, f, E, k, n_shared, PRICHS_DTYPE_BF16, max_tokens, &eng->moe);
  if (rc) {
    delete eng;
    return rc;
  }
  const size_t T = max_tokens, half = eng->hd / 2;
  Carve c;
  const size_t o_wqkv = c.take(2 * prichs_packed_weight_elems(d, eng->qkv_n, PRICHS_DTYPE_BF16));
  const size_t o_wo = c.take(2 * prichs_packed_weight_elems(d, d, PRICHS_DTYPE_BF16));
  const size_t o_in = c.take(4 * d), o_post = c.take(4 * d);
  const size_t o_cos = c.take(4 * max_seq_len * half), o_sin = c.take(4 * max_seq_len * half);
  const size_t o_n1 = c.take(2 * T * d), o_qkv = c.take(2 * T * eng->qkv_n);
  const size_t o_attn = c.take(2 * T * d), o_ao = c.take(2 * T * d), o_x1 = c.take(4 * T * d);
  const size_t o_n2 = c.take(2 * T * d), o_mo = c.take(2 * T * d);

  if (hipGetDevice(&eng->device) != hipSuccess) {
    rc = fail(PRICHS_ERR_HIP, "block_create: no HIP device");
  } else {
    const hipError_t e = hipMalloc(&eng->arena, c.off);
    if (e != hipSuccess) {
      eng->arena = nullptr;
      rc = fail(PRICHS_ERR_CAPACITY, "block_create: hipMalloc(%zu bytes): %s", c.off,
                hipGetErrorString(e));
    }
  }
  if (rc == PRICHS_OK) {
    std::vector<float> cs(max_seq_len * half), sn(max_seq_len * half);
    rc = prichs_rope_cache(max_seq_len, eng->hd, rope_theta, cs.data(), sn.data());
    char *base = static_cast<char *>(eng->arena);
    eng->w_qkv = base + o_wqkv;
    eng->w_o = base + o_wo;
    eng->input_norm = reinterpret_cast<float *>(base + o_in);
    eng->post_norm = reinterpret_cast<float *>(base + o_post);
    eng->rope_cos = reinterpret_cast<float *>(base + o_cos);
    eng->rope_sin = reinterpret_cast<float *>(base + o_sin);
    eng->n1 = base + o_n1;
    eng->qkv = base + o_qkv;
    eng->attn = base + o_attn;
    eng->attn_out = base + o_ao;
    eng->x1 = reinterpret_cast<float *>(base + o_x1);
    eng->n2 = base + o_n2;
    eng->moe_out = base + o_mo;
    if (rc == PRICHS_OK &&
        (hipMemcpy(eng->rope_cos, cs.data(), 4 * cs.size(), hipMemcpyHostToDevice) != hipSuccess ||
         hipMemcpy(eng->rope_sin, sn.data(), 4 * sn.size(), hipMemcpyHostToDevice) != hipSuccess))
      rc = fail(PRICHS_ERR_HIP, "block_create: uploading the RoPE tables failed");
  }
  if (rc != PRICHS_OK) {
    prichs_block_engine_destroy(eng);
    return rc;
  }
  *out = eng;
  return PRICHS_OK;
}

extern "C" int prichs_block_engine_destroy(prichs_block_engine *eng) {
  if (!eng) return PRICHS_OK;
  int rc = prichs_moe_engine_destroy(eng->moe);
  if (eng->arena) {
    int prev = -1;
    (void)hipGetDevice(&prev);
    if (prev != eng->device) (void)hipSetDevice(eng->device);
    if (hipFree(eng->arena) != hipSuccess && rc == PRICHS_OK)
      rc = fail(PRICHS_ERR_HIP, "block_destroy: hipFree failed");
    if (prev >= 0 && prev != eng->device) (void)hipSetDevice(prev);
  }
  delete eng;
  return rc;
}

extern "C" int prichs_block_engine_upload(prichs_block_engine *eng, const float *input_norm,
                                          const float *post_attn_norm, const float *wq,
                                          const float *wk, const float *wv, const float *wo,
                                          const float *w_router, const float *router_bias,
                                          const float *const *gate, const float *const *up,
                                          const float *const *down) {
  PRICHS_REQUIRE(eng != nullptr, "block_upload: null engine");
  PRICHS_REQUIRE(input_norm && post_attn_norm && wq && wk && wv && wo,
                 "block_upload: null pointer argument");
  const size_t d = eng->d, kvw = eng->Hkv * eng->hd, n = eng->qkv_n;
  // [Wq | Wk | Wv] as one [d, n] matrix (reference layout [K, N], K = d).
  std::vector<float> wqkv(d * n);
  for (size_t r = 0; r < d; ++r) {
    std::memcpy(&wqkv[r * n], wq + r * d, 4 * d);
    std::memcpy(&wqkv[r * n + d], wk + r * kvw, 4 * kvw);
    std::memcpy(&wqkv[r * n + d + kvw], wv + r * kvw, 4 * kvw);
  }
  std::vector<uint16_t> p_qkv(prichs_packed_weight_elems(d, n, PRICHS_DTYPE_BF16));
  std::vector<uint16_t> p_o(prichs_packed_weight_elems(d, d, PRICHS_DTYPE_BF16));
  int rc = prichs_pack_weight(wqkv.data(), d, n, PRICHS_DTYPE_BF16, p_qkv.data());
  if (!rc) rc = prichs_pack_weight(wo, d, d, PRICHS_DTYPE_BF16, p_o.data());
  if (!rc) rc = prichs_moe_engine_upload(eng->moe, w_router, router_bias, gate, up, down);
  if (rc) return rc;
  PRICHS_HIP_TRY(hipMemcpy(eng->w_qkv, p_qkv.data(), 2 * p_qkv.size(), hipMemcpyHostToDevice),
                 "block_upload: qkv");
  PRICHS_HIP_TRY(hipMemcpy(eng->w_o, p_o.data(), 2 * p_o.size(), hipMemcpyHostToDevice),
                 "block_upload: o");
  PRICHS_HIP_TRY(hipMemcpy(eng->input_norm, input_norm, 4 * d, hipMemcpyHostToDevice),
                 "block_upload: input_norm");
  PRICHS_HIP_TRY(hipMemcpy(eng->post_norm, post_attn_norm, 4 * d, hipMemcpyHostToDevice),
                 "block_upload: post_attn_norm");
  PRICHS_HIP_TRY(hipDeviceSynchronize(), "block_upload: synchronize");
  eng->uploaded = true;
  return PRICHS_OK;
}

// Block `layer` of a reference weight file (model.rs:312-338): norms and
// attention projections (slots 0..5), then the MoE; every length is checked
// before anything is uploaded.
extern "C" int prichs_block_engine_upload_checkpoint(prichs_block_engine *eng,
                                                     const prichs_checkpoint *ck, size_t layer,
                                                     const float *router_bias) {
  PRICHS_REQUIRE(eng != nullptr && ck != nullptr, "block_upload_checkpoint: null pointer argument");
  if (eng->S != 1)
    return fail(PRICHS_ERR_UNSUPPORTED,
                "block_upload_checkpoint: a checkpoint layer has one shared expert (moe.rs:61), "
                "the engine has n_shared=%zu",
                eng->S);
  const size_t d = eng->d, kvw = eng->Hkv * eng->hd, E = eng->E;
  struct Part {
    int slot;
    size_t len;
    const char *what;
  };
  const Part parts[6] = {{PRICHS_CKPT_INPUT_NORM, d, "input_norm"},
                         {PRICHS_CKPT_Q_PROJ, d * d, "attention.q_proj"},
                         {PRICHS_CKPT_K_PROJ, d * kvw, "attention.k_proj"},
                         {PRICHS_CKPT_V_PROJ, d * kvw, "attention.v_proj"},
                         {PRICHS_CKPT_OUT_PROJ, d * d, "attention.out_proj"},
                         {PRICHS_CKPT_POST_ATTN_NORM, d, "post_attn_norm"}};
  std::vector<float> v[6];
  for (int i = 0; i < 6; ++i)
    if (int rc = checkpoint_read_vec(ck, prichs_checkpoint_block_param(layer, E, parts[i].slot),
                                     parts[i].len, v[i], parts[i].what, layer))
      return rc;
  CheckpointMoe w;
  if (int rc = checkpoint_moe_weights(ck, layer, d, eng->f, E, w)) return rc;
  return prichs_block_engine_upload(eng, v[0].data(), v[5].data(), v[1].data(), v[2].data(),
                                    v[3].data(), v[4].data(), w.router.data(), router_bias,
                                    w.pg.data(), w.pu.data(), w.pd.data());
}

extern "C" int prichs_block_engine_forward(prichs_block_engine *eng, const void *x, size_t batch,
                                           size_t seq_len, size_t pos_offset,
                                           const float *concept_bias, size_t n_concept, void *out,
                                           int out_dtype, void *stream) {
  PRICHS_REQUIRE(eng != nullptr, "block_forward: null engine");
  PRICHS_REQUIRE(dtype_ok(out_dtype), "block_forward: bad out dtype %d", out_dtype);
  if (!eng->uploaded) return fail(PRICHS_ERR_STATE, "block_forward: weights not uploaded");
  const size_t T = batch * seq_len;
  if (T > eng->max_tokens)
    return fail(PRICHS_ERR_CAPACITY, "block_forward: batch*seq_len=%zu exceeds max_tokens=%zu", T,
                eng->max_tokens);
  if (seq_len + pos_offset > eng->cache_rows)
    return fail(PRICHS_ERR_CAPACITY, "block_forward: positions up to %zu exceed max_seq_len=%zu",
                seq_len + pos_offset, eng->cache_rows);
  if (T == 0) {
    eng->last_T = 0;
    return PRICHS_OK;
  }
  PRICHS_REQUIRE(x && out, "block_forward: null pointer argument");
  const size_t d = eng->d, n = eng->qkv_n, kvw = eng->Hkv * eng->hd;
  const int bf = PRICHS_DTYPE_BF16;
  bf16_t *qkv = static_cast<bf16_t *>(eng->qkv);
  int rc;
  if ((rc = prichs_rmsnorm_forward(x, bf, eng->input_norm, eng->n1, bf, nullptr, T, d, eng->eps,
                                   stream)))
    return rc;
  if ((rc = prichs_gemm(eng->n1, d, T, d, eng->w_qkv, n, qkv, n, bf, stream))) return rc;
  // RoPE: the k heads in place (one launch), q inside the attention kernel
  // as it loads its fragments (same bf16 values, one pass over q saved).
  if ((rc = prichs_rope_forward_ld(qkv + d, n, bf, eng->rope_cos, eng->rope_sin, eng->cache_rows,
                                   batch, seq_len, eng->Hkv, eng->hd, pos_offset, 1, stream)))
    return rc;
  if ((rc = attention_forward_impl(qkv, n, qkv + d, n, qkv + d + kvw, n, eng->attn, d, batch,
                                   seq_len, eng->Hq, eng->Hkv, eng->hd, bf, eng->rope_cos,
                                   eng->rope_sin, eng->cache_rows, pos_offset, stream)))
    return rc;
  if ((rc = prichs_gemm(eng->attn, d, T, d, eng->w_o, d, eng->attn_out, d, bf, stream))) return rc;
  if ((rc = add_rmsnorm_forward(x, bf, eng->attn_out, bf, eng->x1, eng->post_norm, eng->n2, T, d,
                                 eng->eps, stream)))
    return rc;
  if ((rc = moe_engine_forward_residual(eng->moe, eng->n2, T, concept_bias, n_concept,
                                       eng->moe_out, eng->x1, out, out_dtype, stream)))
    return rc;
  eng->last_T = T;
  return PRICHS_OK;
}

extern "C" int prichs_block_engine_stash(const prichs_block_engine *eng, prichs_block_stash *out) {
  PRICHS_REQUIRE(eng && out, "block_stash: null pointer argument");
  out->T = eng->last_T;
  out->normed1 = eng->n1;
  out->qkv = eng->qkv;
  out->attn = eng->attn;
  out->attn_out = eng->attn_out;
  out->x1 = eng->x1;
  out->normed2 = eng->n2;
  out->moe_out = eng->moe_out;
  out->moe = eng->moe;
  return PRICHS_OK;
}
