// gpu_model_engine.cpp -- the C++ host mirror of GpuModelEngine over the C ABI
// of libprichs_hip.so.  Each method cites the reference method it mirrors
// (crates/prichs-cuda/src/engine.rs).
#include "gpu_model_engine.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "prichs_hip.h"

namespace prichs_host {

namespace {

[[noreturn]] void bail(const std::string &msg) { throw Error(msg); }

std::string fmt(const char *f, ...) __attribute__((format(printf, 1, 2)));
std::string fmt(const char *f, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, f);
  vsnprintf(buf, sizeof buf, f, ap);
  va_end(ap);
  return buf;
}

void hip_ok(hipError_t e, const char *what) {
  if (e != hipSuccess) bail(fmt("%s failed: %s", what, hipGetErrorString(e)));
}

// A status of the stage entry points -> Error with the library's message.
void lib_ok(int rc, const char *what) {
  if (rc != PRICHS_OK) bail(fmt("%s failed (status %d): %s", what, rc, prichs_last_error()));
}

// The legacy launchers return void and record failures in the last-error slot.
template <typename F> void legacy(const char *what, F &&launch) {
  prichs_clear_error();
  launch();
  const char *e = prichs_last_error();
  if (e != nullptr && e[0] != 0) bail(fmt("%s failed: %s", what, e));
}

// Leading dimension of padded GEMM operands: the f32 kernel takes K and N in
// multiples of 16 (zero padding leaves every sum unchanged).
size_t ld16(size_t n) { return (n + 15) / 16 * 16; }

template <typename T> T *dev_alloc(size_t elems, const char *what) {
  void *p = nullptr;
  hip_ok(hipMalloc(&p, std::max<size_t>(elems, 1) * sizeof(T)), what);
  return static_cast<T *>(p);
}

// rows x cols host matrix -> device rows with leading dimension ld, pad zero.
void h2d_padded(float *dst, size_t ld, const float *src, size_t rows, size_t cols) {
  hip_ok(hipMemset(dst, 0, rows * ld * sizeof(float)), "hipMemset");
  hip_ok(hipMemcpy2D(dst, ld * sizeof(float), src, cols * sizeof(float), cols * sizeof(float),
                     rows, hipMemcpyHostToDevice),
         "hipMemcpy2D H2D");
}

std::vector<float> d2h_rows(const float *src, size_t ld, size_t rows, size_t cols) {
  std::vector<float> out(rows * cols);
  if (rows * cols == 0) return out;
  hip_ok(hipMemcpy2D(out.data(), cols * sizeof(float), src, ld * sizeof(float),
                     cols * sizeof(float), rows, hipMemcpyDeviceToHost),
         "hipMemcpy2D D2H");
  return out;
}

}  // namespace

Checkpoint load_checkpoint(const std::string &path) {
  prichs_checkpoint *ck = nullptr;
  lib_ok(prichs_checkpoint_open(path.c_str(), &ck), "load_checkpoint");
  Checkpoint out;
  try {
    size_t n = 0;
    int format = 0;
    lib_ok(prichs_checkpoint_info(ck, &out.step, &out.loss, &n, &format), "load_checkpoint");
    if (format != 2)
      bail(fmt("load_checkpoint: %s is a legacy PRICHS_W file (embedding and final norm only)",
               path.c_str()));
    out.params.resize(n);
    for (size_t i = 0; i < n; ++i) {
      size_t len = 0;
      lib_ok(prichs_checkpoint_param_len(ck, i, &len), "load_checkpoint");
      out.params[i].resize(len);
      lib_ok(prichs_checkpoint_read(ck, i, out.params[i].data(), len), "load_checkpoint");
    }
  } catch (...) {
    prichs_checkpoint_close(ck);
    throw;
  }
  prichs_checkpoint_close(ck);
  return out;
}

size_t block_param_index(size_t layer, size_t E, size_t slot) {
  const size_t i = prichs_checkpoint_block_param(layer, E, slot);
  if (i == (size_t)-1) bail(fmt("block_param_index: slot %zu outside a block of %zu", slot, 10 + 3 * E));
  return i;
}

struct GpuModelEngine::PackedGemm {
  size_t Kp = 0, Np = 0;
  float *dev = nullptr;
};

// engine.rs:363-649.
GpuModelEngine::GpuModelEngine(const std::vector<std::tuple<size_t, size_t, bool>> &param_shapes,
                               const Capacity &cap)
    : cap_(cap) {
  size_t offset = 0;
  meta_.reserve(param_shapes.size());
  for (size_t id = 0; id < param_shapes.size(); ++id) {
    ParamMetadata m;
    m.id = id;
    m.offset = offset;
    m.rows = std::get<0>(param_shapes[id]);
    m.cols = std::get<1>(param_shapes[id]);
    m.len = m.rows * m.cols;
    m.apply_weight_decay = std::get<2>(param_shapes[id]);
    meta_.push_back(m);
    offset += m.len;
  }
  packed_.assign(meta_.size(), nullptr);
  try {
    dev_weights_ = dev_alloc<float>(offset, "hipMalloc(dev_weights)");
    dev_act_in_ = dev_alloc<float>(cap_.act_in, "hipMalloc(act_in)");
    dev_act_out_ = dev_alloc<float>(cap_.act_out, "hipMalloc(act_out)");
    dev_x_ = dev_alloc<float>(cap_.act_in, "hipMalloc(exp_x)");
    dev_gate_ = dev_alloc<float>(cap_.moe_dim, "hipMalloc(gate)");
    dev_up_ = dev_alloc<float>(cap_.moe_dim, "hipMalloc(up)");
    dev_act_ = dev_alloc<float>(cap_.moe_dim, "hipMalloc(act)");
    dev_out_ = dev_alloc<float>(cap_.act_in, "hipMalloc(exp_out)");
    dev_moe_out_ = dev_alloc<float>(cap_.act_in, "hipMalloc(moe_out)");
    dev_rstd_ = dev_alloc<float>(cap_.max_rows, "hipMalloc(rstd)");
    dev_cos_ = dev_alloc<float>(cap_.rope_cache, "hipMalloc(cos)");
    dev_sin_ = dev_alloc<float>(cap_.rope_cache, "hipMalloc(sin)");
    dev_idx_ = dev_alloc<int32_t>(cap_.max_rows, "hipMalloc(exp_indices)");
    dev_w_ = dev_alloc<float>(cap_.max_rows, "hipMalloc(exp_weights)");
  } catch (...) {
    release();
    throw;
  }
}

GpuModelEngine::~GpuModelEngine() { release(); }

void GpuModelEngine::release() {
  for (MoeLayer &l : layers_)
    if (l.eng != nullptr) prichs_moe_engine_destroy(l.eng);
  layers_.clear();
  for (PackedGemm *p : packed_) {
    if (p != nullptr) (void)hipFree(p->dev);
    delete p;
  }
  packed_.clear();
  for (void *p : {(void *)dev_weights_, (void *)dev_act_in_, (void *)dev_act_out_, (void *)dev_x_,
                  (void *)dev_gate_, (void *)dev_up_, (void *)dev_act_, (void *)dev_out_,
                  (void *)dev_moe_out_, (void *)dev_rstd_, (void *)dev_cos_, (void *)dev_sin_,
                  (void *)dev_idx_, (void *)dev_w_, (void *)dev_q_, (void *)dev_k_,
                  (void *)dev_v_, (void *)dev_cat_, (void *)dev_probs_})
    if (p != nullptr) (void)hipFree(p);
  dev_q_ = dev_k_ = dev_v_ = dev_cat_ = dev_probs_ = nullptr;
  dev_weights_ = dev_act_in_ = dev_act_out_ = dev_x_ = dev_gate_ = dev_up_ = dev_act_ = nullptr;
  dev_out_ = dev_moe_out_ = dev_rstd_ = dev_cos_ = dev_sin_ = dev_w_ = nullptr;
  dev_idx_ = nullptr;
}

void GpuModelEngine::check_param(size_t id, const char *who) const {
  if (id >= meta_.size()) bail(fmt("%s: param id %zu out of range (%zu params)", who, id, meta_.size()));
}

// engine.rs:668-689.
void GpuModelEngine::upload_weights(const std::vector<std::vector<float>> &param_slices) {
  if (param_slices.size() != meta_.size())
    bail(fmt("param_slices count %zu != meta count %zu", param_slices.size(), meta_.size()));
  for (const ParamMetadata &m : meta_) {
    if (param_slices[m.id].size() != m.len)
      bail(fmt("Param %zu length mismatch: host %zu != meta %zu", m.id, param_slices[m.id].size(),
               m.len));
    hip_ok(hipMemcpy(dev_weights_ + m.offset, param_slices[m.id].data(), m.len * sizeof(float),
                     hipMemcpyHostToDevice),
           "hipMemcpy upload");
  }
  // Packed GEMM copies are rebuilt from the new weights on next use.
  for (PackedGemm *&p : packed_) {
    if (p != nullptr) (void)hipFree(p->dev);
    delete p;
    p = nullptr;
  }
  hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
}

// engine.rs:691-708.
void GpuModelEngine::download_weights(std::vector<std::vector<float>> &param_slices) const {
  if (param_slices.size() != meta_.size())
    bail(fmt("param_slices count %zu != meta count %zu", param_slices.size(), meta_.size()));
  for (const ParamMetadata &m : meta_) {
    param_slices[m.id].resize(m.len);
    hip_ok(hipMemcpy(param_slices[m.id].data(), dev_weights_ + m.offset, m.len * sizeof(float),
                     hipMemcpyDeviceToHost),
           "hipMemcpy download");
  }
}

// The f32 weight [K, N] of a parameter, zero-padded to [Kp, Np] and packed
// for prichs_gemm (built once per upload).
const GpuModelEngine::PackedGemm &GpuModelEngine::packed(size_t param_id) {
  if (packed_[param_id] != nullptr) return *packed_[param_id];
  const ParamMetadata &m = meta_[param_id];
  const size_t Kp = ld16(m.rows), Np = ld16(m.cols);
  std::vector<float> w(m.len), wpad(Kp * Np, 0.0f);
  hip_ok(hipMemcpy(w.data(), dev_weights_ + m.offset, m.len * sizeof(float),
                   hipMemcpyDeviceToHost),
         "hipMemcpy weights");
  for (size_t k = 0; k < m.rows; ++k)
    std::copy(w.begin() + k * m.cols, w.begin() + (k + 1) * m.cols, wpad.begin() + k * Np);
  std::vector<float> host(prichs_packed_weight_elems(Kp, Np, PRICHS_DTYPE_F32));
  lib_ok(prichs_pack_weight(wpad.data(), Kp, Np, PRICHS_DTYPE_F32, host.data()),
         "prichs_pack_weight");
  auto *p = new PackedGemm;
  p->Kp = Kp;
  p->Np = Np;
  try {
    p->dev = dev_alloc<float>(host.size(), "hipMalloc(packed weight)");
    hip_ok(hipMemcpy(p->dev, host.data(), host.size() * sizeof(float), hipMemcpyHostToDevice),
           "hipMemcpy packed weight");
  } catch (...) {
    delete p;
    throw;
  }
  packed_[param_id] = p;
  return *p;
}

// out_dev[m, Np] (leading dimension ldo) = x_dev[m, Kp] (ldx) @ W[param_id].
void GpuModelEngine::gemm_dev(size_t param_id, const float *x_dev, size_t ldx, float *out_dev,
                              size_t ldo, size_t m) {
  const PackedGemm &p = packed(param_id);
  lib_ok(prichs_gemm(x_dev, ldx, m, p.Kp, p.dev, p.Np, out_dev, ldo, PRICHS_DTYPE_F32, nullptr),
         "prichs_gemm");
}

// engine.rs:757-826.
void GpuModelEngine::forward_gemm(size_t param_id, const std::vector<float> &x,
                                  std::vector<float> &out, size_t m, size_t k, size_t n) {
  check_param(param_id, "forward_gemm");
  const ParamMetadata &meta = meta_[param_id];
  if (meta.rows != k || meta.cols != n)
    bail(fmt("Param %zu shape mismatch: expected [%zu, %zu], meta is [%zu, %zu]", param_id, k, n,
             meta.rows, meta.cols));
  const size_t Kp = ld16(k), Np = ld16(n);
  if (m * Kp > cap_.act_in || m * Np > cap_.act_out)
    bail("Activation dimensions exceed preallocated VRAM workspace");
  if (x.size() < m * k || out.size() < m * n)
    bail(fmt("forward_gemm: x holds %zu < %zu or out %zu < %zu elements", x.size(), m * k,
             out.size(), m * n));
  if (m == 0) return;
  h2d_padded(dev_act_in_, Kp, x.data(), m, k);
  act_in_ld_ = 0;  // normed2 no longer resident
  gemm_dev(param_id, dev_act_in_, Kp, dev_act_out_, Np, m);
  const std::vector<float> o = d2h_rows(dev_act_out_, Np, m, n);
  std::copy(o.begin(), o.end(), out.begin());
  hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
}

// engine.rs:1788-1846.
void GpuModelEngine::gpu_rmsnorm_forward(const std::vector<float> &x, size_t param_id,
                                         std::vector<float> &out, std::vector<float> &rstd,
                                         size_t seq_len, size_t hidden_dim, float eps) {
  check_param(param_id, "gpu_rmsnorm_forward");
  const ParamMetadata &meta = meta_[param_id];
  if (meta.len != hidden_dim)
    bail(fmt("RMSNorm param %zu len mismatch: %zu != %zu", param_id, meta.len, hidden_dim));
  const size_t total = seq_len * hidden_dim;
  if (total > cap_.act_in || total > cap_.act_out || seq_len > cap_.max_rows)
    bail("RMSNorm dimensions exceed workspace capacity");
  if (x.size() < total || out.size() < total || rstd.size() < seq_len)
    bail("gpu_rmsnorm_forward: host slice shorter than seq_len * hidden_dim");
  if (total == 0) return;
  hip_ok(hipMemcpy(dev_act_in_, x.data(), total * sizeof(float), hipMemcpyHostToDevice),
         "hipMemcpy H2D");
  act_in_ld_ = 0;
  lib_ok(prichs_rmsnorm_forward(dev_act_in_, PRICHS_DTYPE_F32, dev_weights_ + meta.offset,
                                dev_act_out_, PRICHS_DTYPE_F32, dev_rstd_, seq_len, hidden_dim,
                                eps, nullptr),
         "prichs_rmsnorm_forward");
  hip_ok(hipMemcpy(out.data(), dev_act_out_, total * sizeof(float), hipMemcpyDeviceToHost),
         "hipMemcpy D2H");
  hip_ok(hipMemcpy(rstd.data(), dev_rstd_, seq_len * sizeof(float), hipMemcpyDeviceToHost),
         "hipMemcpy D2H");
}

// engine.rs:1162-1179.
void GpuModelEngine::upload_rope_cache(const std::vector<float> &cos_cache,
                                       const std::vector<float> &sin_cache) {
  if (cos_cache.size() != sin_cache.size()) bail("cos_cache and sin_cache must have equal length");
  if (cos_cache.size() > cap_.rope_cache)
    bail(fmt("RoPE cache length %zu exceeds capacity %zu", cos_cache.size(), cap_.rope_cache));
  const size_t bytes = cos_cache.size() * sizeof(float);
  hip_ok(hipMemcpy(dev_cos_, cos_cache.data(), bytes, hipMemcpyHostToDevice), "hipMemcpy cos");
  hip_ok(hipMemcpy(dev_sin_, sin_cache.data(), bytes, hipMemcpyHostToDevice), "hipMemcpy sin");
  rope_len_ = cos_cache.size();
}

// engine.rs:1181-1405.
AttentionOut GpuModelEngine::gpu_batched_attention_forward(
    const std::vector<float> &normed1, size_t q_id, size_t k_id, size_t v_id, size_t out_id,
    std::vector<float> &attn_out, size_t seq_len, size_t num_heads, size_t num_kv_heads,
    size_t head_dim) {
  const size_t hidden = num_heads * head_dim, kv = num_kv_heads * head_dim;
  // The reference's checks (engine.rs:1197-1208), then the weight shapes.
  if (normed1.size() != seq_len * hidden)
    bail(fmt("normed1 length mismatch: %zu != %zu", normed1.size(), seq_len * hidden));
  if (attn_out.size() != seq_len * hidden)
    bail(fmt("attn_out length mismatch: %zu != %zu", attn_out.size(), seq_len * hidden));
  if (seq_len * hidden > cap_.attn_vec) bail("Attention dimensions exceed attn_vec_capacity");
  if (num_heads * seq_len * seq_len > cap_.attn_scores)
    bail("Attention scores dimensions exceed attn_scores_capacity");
  if (num_kv_heads == 0 || num_heads % num_kv_heads != 0)
    bail(fmt("num_heads=%zu is not a multiple of num_kv_heads=%zu", num_heads, num_kv_heads));
  for (size_t id : {q_id, k_id, v_id, out_id}) check_param(id, "gpu_batched_attention_forward");
  const ParamMetadata &mq = meta_[q_id], &mk = meta_[k_id], &mv = meta_[v_id],
                      &mo = meta_[out_id];
  if (mq.rows != hidden || mq.cols != hidden || mk.rows != hidden || mk.cols != kv ||
      mv.rows != hidden || mv.cols != kv || mo.rows != hidden || mo.cols != hidden)
    bail("attention weight shapes do not match the head layout");
  if (head_dim % 2 != 0) bail(fmt("head_dim %zu must be even for RoPE", head_dim));
  if (seq_len * (head_dim / 2) > rope_len_)
    bail(fmt("seq_len %zu needs %zu RoPE cache entries; %zu uploaded", seq_len,
             seq_len * (head_dim / 2), rope_len_));
  if (dev_q_ == nullptr) {
    dev_q_ = dev_alloc<float>(cap_.attn_vec, "hipMalloc(q)");
    dev_k_ = dev_alloc<float>(cap_.attn_vec, "hipMalloc(k)");
    dev_v_ = dev_alloc<float>(cap_.attn_vec, "hipMalloc(v)");
    dev_cat_ = dev_alloc<float>(cap_.attn_vec, "hipMalloc(concat)");
    dev_probs_ = dev_alloc<float>(cap_.attn_scores, "hipMalloc(scores)");
  }
  if (seq_len * hidden > cap_.act_in || seq_len * hidden > cap_.act_out)
    bail("Attention dimensions exceed the activation capacity");
  const size_t q_bytes = seq_len * hidden * sizeof(float), kv_bytes = seq_len * kv * sizeof(float);
  hip_ok(hipMemcpy(dev_act_in_, normed1.data(), q_bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
  lib_ok(prichs_matmul_f32(PRICHS_MATMUL_AB, dev_act_in_, dev_weights_ + mq.offset, dev_q_,
                           seq_len, hidden, hidden, nullptr), "Q projection");
  lib_ok(prichs_matmul_f32(PRICHS_MATMUL_AB, dev_act_in_, dev_weights_ + mk.offset, dev_k_,
                           seq_len, hidden, kv, nullptr), "K projection");
  lib_ok(prichs_matmul_f32(PRICHS_MATMUL_AB, dev_act_in_, dev_weights_ + mv.offset, dev_v_,
                           seq_len, hidden, kv, nullptr), "V projection");
  // RoPE like the reference's launch_rope (positions 0.., sign +1).
  lib_ok(prichs_rope_forward(dev_q_, PRICHS_DTYPE_F32, dev_cos_, dev_sin_, seq_len, 1, seq_len,
                             num_heads, head_dim, 0, 1, nullptr), "RoPE Q");
  lib_ok(prichs_rope_forward(dev_k_, PRICHS_DTYPE_F32, dev_cos_, dev_sin_, seq_len, 1, seq_len,
                             num_kv_heads, head_dim, 0, 1, nullptr), "RoPE K");
  lib_ok(prichs_attention_probs_f32(dev_q_, dev_k_, dev_v_, dev_probs_, dev_cat_, seq_len,
                                    num_heads, num_kv_heads, head_dim, nullptr), "attention");
  lib_ok(prichs_matmul_f32(PRICHS_MATMUL_AB, dev_cat_, dev_weights_ + mo.offset, dev_act_out_,
                           seq_len, hidden, hidden, nullptr), "out projection");
  std::vector<float> q_rope(seq_len * hidden), k_rope(seq_len * kv), v(seq_len * kv),
      probs(num_heads * seq_len * seq_len), concat(seq_len * hidden);
  hip_ok(hipMemcpy(attn_out.data(), dev_act_out_, q_bytes, hipMemcpyDeviceToHost), "D2H out");
  hip_ok(hipMemcpy(q_rope.data(), dev_q_, q_bytes, hipMemcpyDeviceToHost), "D2H q");
  hip_ok(hipMemcpy(k_rope.data(), dev_k_, kv_bytes, hipMemcpyDeviceToHost), "D2H k");
  hip_ok(hipMemcpy(v.data(), dev_v_, kv_bytes, hipMemcpyDeviceToHost), "D2H v");
  hip_ok(hipMemcpy(probs.data(), dev_probs_, probs.size() * sizeof(float), hipMemcpyDeviceToHost),
         "D2H probs");
  hip_ok(hipMemcpy(concat.data(), dev_cat_, q_bytes, hipMemcpyDeviceToHost), "D2H concat");
  hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
  return AttentionOut{std::move(q_rope), std::move(k_rope), std::move(v), std::move(probs),
                      std::move(concat)};
}

// engine.rs:1917-2051.
SharedOut GpuModelEngine::gpu_moe_forward_shared(const std::vector<float> &normed2,
                                                 size_t gate_id, size_t up_id, size_t down_id,
                                                 size_t seq_len, size_t hidden_dim,
                                                 size_t intermediate_dim) {
  for (size_t id : {gate_id, up_id, down_id}) check_param(id, "gpu_moe_forward_shared");
  const size_t T = seq_len, d = hidden_dim, f = intermediate_dim;
  const ParamMetadata &g = meta_[gate_id], &u = meta_[up_id], &dn = meta_[down_id];
  if (g.rows != d || g.cols != f || u.rows != d || u.cols != f || dn.rows != f || dn.cols != d)
    bail(fmt("MoE shared weights must be gate/up [%zu, %zu] and down [%zu, %zu]", d, f, f, d));
  const size_t dp = ld16(d), fp = ld16(f);
  if (T * dp > cap_.act_in || T * fp > cap_.moe_dim) bail("MoE shared dimensions exceed workspace");
  if (normed2.size() < T * d) bail("gpu_moe_forward_shared: normed2 shorter than seq_len * hidden_dim");
  if (T == 0) return {};
  h2d_padded(dev_act_in_, dp, normed2.data(), T, d);
  act_in_ld_ = dp;
  gemm_dev(gate_id, dev_act_in_, dp, dev_gate_, fp, T);
  gemm_dev(up_id, dev_act_in_, dp, dev_up_, fp, T);
  legacy("launch_swiglu_forward",
         [&] { launch_swiglu_forward(dev_gate_, dev_up_, dev_act_, T * fp, nullptr); });
  // The shared expert's output starts the accumulator (beta = 0 in the reference).
  gemm_dev(down_id, dev_act_, fp, dev_moe_out_, dp, T);
  moe_rows_ = T;
  moe_ld_ = dp;
  moe_d_ = d;
  SharedOut r{d2h_rows(dev_gate_, fp, T, f), d2h_rows(dev_up_, fp, T, f),
              d2h_rows(dev_act_, fp, T, f), d2h_rows(dev_moe_out_, dp, T, d)};
  hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
  return r;
}

// engine.rs:2054-2223.
ExpertOut GpuModelEngine::gpu_moe_forward_expert(const std::vector<int32_t> &token_indices,
                                                 const std::vector<float> &weights,
                                                 size_t gate_id, size_t up_id, size_t down_id,
                                                 size_t hidden_dim, size_t intermediate_dim) {
  const size_t n = token_indices.size();
  if (n == 0) return {};
  for (size_t id : {gate_id, up_id, down_id}) check_param(id, "gpu_moe_forward_expert");
  const size_t d = hidden_dim, f = intermediate_dim;
  const ParamMetadata &g = meta_[gate_id], &u = meta_[up_id], &dn = meta_[down_id];
  if (g.rows != d || g.cols != f || u.rows != d || u.cols != f || dn.rows != f || dn.cols != d)
    bail(fmt("MoE expert weights must be gate/up [%zu, %zu] and down [%zu, %zu]", d, f, f, d));
  if (weights.size() != n)
    bail(fmt("gpu_moe_forward_expert: %zu weights for %zu tokens", weights.size(), n));
  if (act_in_ld_ == 0 || moe_d_ != d)
    bail("gpu_moe_forward_expert: run gpu_moe_forward_shared on this batch first");
  const size_t dp = ld16(d), fp = ld16(f);
  if (n > cap_.max_rows || n * dp > cap_.act_in || n * fp > cap_.moe_dim)
    bail("MoE expert dimensions exceed workspace");
  for (int32_t t : token_indices)
    if (t < 0 || (size_t)t >= moe_rows_)
      bail(fmt("gpu_moe_forward_expert: token index %d outside [0, %zu)", t, moe_rows_));
  hip_ok(hipMemcpy(dev_idx_, token_indices.data(), n * sizeof(int32_t), hipMemcpyHostToDevice),
         "hipMemcpy indices");
  hip_ok(hipMemcpy(dev_w_, weights.data(), n * sizeof(float), hipMemcpyHostToDevice),
         "hipMemcpy weights");
  legacy("launch_moe_gather",
         [&] { launch_moe_gather(dev_act_in_, dev_idx_, dev_x_, n, dp, nullptr); });
  gemm_dev(gate_id, dev_x_, dp, dev_gate_, fp, n);
  gemm_dev(up_id, dev_x_, dp, dev_up_, fp, n);
  legacy("launch_swiglu_forward",
         [&] { launch_swiglu_forward(dev_gate_, dev_up_, dev_act_, n * fp, nullptr); });
  gemm_dev(down_id, dev_act_, fp, dev_out_, dp, n);
  legacy("launch_moe_scatter_add", [&] {
    launch_moe_scatter_add(dev_out_, dev_idx_, dev_w_, dev_moe_out_, n, dp, nullptr);
  });
  ExpertOut r{d2h_rows(dev_x_, dp, n, d), d2h_rows(dev_gate_, fp, n, f),
              d2h_rows(dev_up_, fp, n, f), d2h_rows(dev_act_, fp, n, f),
              d2h_rows(dev_out_, dp, n, d)};
  hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
  return r;
}

// engine.rs:2226-2239.
void GpuModelEngine::gpu_moe_finalize_forward(std::vector<float> &total_out) const {
  if (total_out.size() < moe_rows_ * moe_d_)
    bail(fmt("gpu_moe_finalize_forward: output holds %zu < %zu elements", total_out.size(),
             moe_rows_ * moe_d_));
  const std::vector<float> o = d2h_rows(dev_moe_out_, moe_ld_, moe_rows_, moe_d_);
  std::copy(o.begin(), o.end(), total_out.begin());
}

// engine.rs:2694-2702.
void GpuModelEngine::sync_stream() const {
  hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
}

size_t GpuModelEngine::create_moe_layer(
    size_t router_id, const std::vector<float> &router_bias, size_t shared_gate, size_t shared_up,
    size_t shared_down, const std::vector<std::tuple<size_t, size_t, size_t>> &experts,
    size_t top_k, int dtype, size_t max_tokens) {
  check_param(router_id, "create_moe_layer");
  const size_t E = experts.size();
  const ParamMetadata &r = meta_[router_id];
  if (r.cols != E) bail(fmt("create_moe_layer: router has %zu columns for %zu experts", r.cols, E));
  if (!router_bias.empty() && router_bias.size() != E)
    bail(fmt("create_moe_layer: router_bias has %zu entries for %zu experts", router_bias.size(), E));
  const size_t d = r.rows;
  std::vector<std::tuple<size_t, size_t, size_t>> all{{shared_gate, shared_up, shared_down}};
  all.insert(all.end(), experts.begin(), experts.end());
  const size_t f = meta_.at(shared_gate).cols;
  for (const auto &e : all) {
    for (size_t id : {std::get<0>(e), std::get<1>(e), std::get<2>(e)}) check_param(id, "create_moe_layer");
    const ParamMetadata &g = meta_[std::get<0>(e)], &u = meta_[std::get<1>(e)],
                        &dn = meta_[std::get<2>(e)];
    if (g.rows != d || g.cols != f || u.rows != d || u.cols != f || dn.rows != f || dn.cols != d)
      bail(fmt("create_moe_layer: expert weights must be gate/up [%zu, %zu], down [%zu, %zu]", d,
               f, f, d));
  }
  MoeLayer layer;
  layer.d = d;
  layer.E = E;
  layer.dtype = dtype;
  lib_ok(prichs_moe_engine_create(d, f, E, top_k, 1, dtype, max_tokens, &layer.eng),
         "prichs_moe_engine_create");
  try {
    auto host = [&](size_t id) {
      const ParamMetadata &m = meta_[id];
      std::vector<float> v(m.len);
      hip_ok(hipMemcpy(v.data(), dev_weights_ + m.offset, m.len * sizeof(float),
                       hipMemcpyDeviceToHost),
             "hipMemcpy weights");
      return v;
    };
    std::vector<std::vector<float>> g, u, dn;
    for (const auto &e : all) {
      g.push_back(host(std::get<0>(e)));
      u.push_back(host(std::get<1>(e)));
      dn.push_back(host(std::get<2>(e)));
    }
    std::vector<const float *> gp, up, dp;
    for (size_t i = 0; i < all.size(); ++i) {
      gp.push_back(g[i].data());
      up.push_back(u[i].data());
      dp.push_back(dn[i].data());
    }
    const std::vector<float> wr = host(router_id);
    lib_ok(prichs_moe_engine_upload(layer.eng, wr.data(),
                                    router_bias.empty() ? nullptr : router_bias.data(), gp.data(),
                                    up.data(), dp.data()),
           "prichs_moe_engine_upload");
  } catch (...) {
    prichs_moe_engine_destroy(layer.eng);
    throw;
  }
  layers_.push_back(layer);
  return layers_.size() - 1;
}

void GpuModelEngine::gpu_moe_forward(size_t layer_id, const void *x_dev, size_t T, void *out_dev,
                                     void *stream) {
  if (layer_id >= layers_.size()) bail(fmt("gpu_moe_forward: no MoE layer %zu", layer_id));
  const MoeLayer &l = layers_[layer_id];
  lib_ok(prichs_moe_engine_forward(l.eng, x_dev, T, nullptr, 0, out_dev, l.dtype, stream),
         "prichs_moe_engine_forward");
}

void GpuModelEngine::set_moe_router_bias(size_t layer_id, const std::vector<float> &router_bias) {
  if (layer_id >= layers_.size()) bail(fmt("set_moe_router_bias: no MoE layer %zu", layer_id));
  const MoeLayer &l = layers_[layer_id];
  if (router_bias.size() != l.E)
    bail(fmt("set_moe_router_bias: %zu entries for %zu experts", router_bias.size(), l.E));
  lib_ok(prichs_moe_engine_set_router_bias(l.eng, router_bias.data()),
         "prichs_moe_engine_set_router_bias");
}

void GpuModelEngine::update_moe_router_bias(size_t layer_id, float gamma, void *stream) {
  if (layer_id >= layers_.size()) bail(fmt("update_moe_router_bias: no MoE layer %zu", layer_id));
  lib_ok(prichs_moe_engine_update_router_bias(layers_[layer_id].eng, gamma, stream),
         "prichs_moe_engine_update_router_bias");
}

std::vector<float> GpuModelEngine::moe_router_bias(size_t layer_id) const {
  if (layer_id >= layers_.size()) bail(fmt("moe_router_bias: no MoE layer %zu", layer_id));
  std::vector<float> b(layers_[layer_id].E);
  lib_ok(prichs_moe_engine_get_router_bias(layers_[layer_id].eng, b.data()),
         "prichs_moe_engine_get_router_bias");
  return b;
}

// ---- GpuWorkspace and the host-slice GEMMs (cublas.rs:46-327) -------------
namespace {
void need(const std::vector<float> &v, size_t elems, const char *what) {
  if (v.size() < elems) bail(fmt("%s holds %zu elements, %zu needed", what, v.size(), elems));
}
}  // namespace

GpuWorkspace::GpuWorkspace(size_t a_bytes, size_t b_bytes, size_t c_bytes) {
  lib_ok(prichs_gpu_workspace_create(a_bytes, b_bytes, c_bytes, &ws_), "GpuWorkspace::new");
}

GpuWorkspace::GpuWorkspace(prichs_gpu_workspace *borrowed) : ws_(borrowed), owned_(false) {}

GpuWorkspace::~GpuWorkspace() {
  if (owned_ && ws_) (void)prichs_gpu_workspace_destroy(ws_);
}

void GpuWorkspace::matmul(const std::vector<float> &a, const std::vector<float> &b,
                          std::vector<float> &c, size_t m, size_t k, size_t n) const {
  need(a, m * k, "a");
  need(b, k * n, "b");
  need(c, m * n, "c");
  lib_ok(prichs_gpu_workspace_matmul(ws_, a.data(), b.data(), c.data(), m, k, n), "matmul");
}

void GpuWorkspace::matmul_at_b(const std::vector<float> &a, const std::vector<float> &b,
                               std::vector<float> &dw, size_t m, size_t k, size_t n) const {
  need(a, m * k, "a");
  need(b, m * n, "b");
  need(dw, k * n, "dw");
  lib_ok(prichs_gpu_workspace_matmul_at_b(ws_, a.data(), b.data(), dw.data(), m, k, n),
         "matmul_at_b");
}

void GpuWorkspace::matmul_a_bt(const std::vector<float> &dy, const std::vector<float> &w,
                               std::vector<float> &dx, size_t m, size_t k, size_t n) const {
  need(dy, m * k, "dy");
  need(w, n * k, "w");
  need(dx, m * n, "dx");
  lib_ok(prichs_gpu_workspace_matmul_a_bt(ws_, dy.data(), w.data(), dx.data(), m, k, n),
         "matmul_a_bt");
}

GpuWorkspace *get_gpu_workspace() {
  static GpuWorkspace *wrapped = nullptr;
  static std::mutex mu;
  std::lock_guard<std::mutex> lock(mu);
  if (wrapped == nullptr) {
    prichs_gpu_workspace *ws = prichs_get_gpu_workspace();
    if (ws == nullptr) return nullptr;
    wrapped = new GpuWorkspace(ws);
  }
  return wrapped;
}

void matmul_gpu(const std::vector<float> &a, const std::vector<float> &b, std::vector<float> &c,
                size_t m, size_t k, size_t n) {
  need(a, m * k, "a");
  need(b, k * n, "b");
  need(c, m * n, "c");
  lib_ok(prichs_matmul_gpu(a.data(), b.data(), c.data(), m, k, n), "matmul_gpu");
}

void matmul_at_b_gpu(const std::vector<float> &a, const std::vector<float> &b,
                     std::vector<float> &dw, size_t m, size_t k, size_t n) {
  need(a, m * k, "a");
  need(b, m * n, "b");
  need(dw, k * n, "dw");
  lib_ok(prichs_matmul_at_b_gpu(a.data(), b.data(), dw.data(), m, k, n), "matmul_at_b_gpu");
}

void matmul_a_bt_gpu(const std::vector<float> &dy, const std::vector<float> &w,
                     std::vector<float> &dx, size_t m, size_t k, size_t n) {
  need(dy, m * k, "dy");
  need(w, n * k, "w");
  need(dx, m * n, "dx");
  lib_ok(prichs_matmul_a_bt_gpu(dy.data(), w.data(), dx.data(), m, k, n), "matmul_a_bt_gpu");
}

}  // namespace prichs_host
