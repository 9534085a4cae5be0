// gpu_model_engine.hpp -- C++ host mirror of the reference's GpuModelEngine
// hot-path interface (crates/prichs-cuda/src/engine.rs), over the C ABI of
// libprichs_hip.so (include/prichs_hip.h).
//
// The reference engine is Rust; no Rust toolchain exists in this build, so
// this mirror keeps its method names, argument meaning and error behaviour in
// C++: a parameter registry over one flat f32 device buffer
// (ParamMetadata, engine.rs:274-282), host slices in and host vectors out,
// fixed workspace capacities checked before any device work, and every
// failure reported as an error value rather than a crash (Rust's
// anyhow::bail! becomes a thrown prichs_host::Error here).
//
// The methods that mirror the reference are the compatibility path (they
// copy across PCIe like the originals).  gpu_moe_forward is the fast path:
// the whole MoE layer on device buffers through the library's MoE engine.
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <tuple>
#include <vector>

struct prichs_moe_engine;
struct prichs_gpu_workspace;

namespace prichs_host {

// anyhow::Error of the reference: a message, thrown where Rust returns Err.
class Error : public std::runtime_error {
 public:
  explicit Error(const std::string &msg) : std::runtime_error(msg) {}
};

// engine.rs:274-282.
struct ParamMetadata {
  size_t id = 0;
  size_t offset = 0;  // in f32 elements of the flat weight buffer
  size_t len = 0;
  size_t rows = 0;
  size_t cols = 0;
  bool apply_weight_decay = false;
};

// Workspace sizes in f32 elements (the reference fixes them in new(),
// engine.rs:363-649).  The defaults cover T = 16384 rows at d = 1536 and
// f = 1280; configuration 2 of the benchmark fits.
struct Capacity {
  size_t act_in = 16384 * 1536;   // normed2 / GEMM input
  size_t act_out = 16384 * 2560;  // GEMM output
  size_t moe_dim = 16384 * 1280;  // [rows, f] intermediates
  size_t rope_cache = 4096 * 64;  // cos / sin entries
  size_t max_rows = 16384;        // RMSNorm rows (rstd)
  // Attention (engine.rs:421-424): [T, H * hd] vectors and the [H, T, T]
  // scores; allocated on the first gpu_batched_attention_forward.
  size_t attn_vec = 4 * 1024 * 1024;
  size_t attn_scores = 32 * 1024 * 1024;
};

// (x, gate, up, act, out) of gpu_moe_forward_expert; the shared form has no x.
using SharedOut = std::tuple<std::vector<float>, std::vector<float>, std::vector<float>,
                             std::vector<float>>;
using ExpertOut = std::tuple<std::vector<float>, std::vector<float>, std::vector<float>,
                             std::vector<float>, std::vector<float>>;
// (q after RoPE, k after RoPE, v, probabilities [H, T, T], heads concatenated)
// of gpu_batched_attention_forward.
using AttentionOut = std::tuple<std::vector<float>, std::vector<float>, std::vector<float>,
                                std::vector<float>, std::vector<float>>;

// Model::load_checkpoint (crates/prichs-model/src/model.rs:1673-1736) for a
// PRICHS02 file, through the library's reader: every parameter in the order
// of get_parameter_tensors (model.rs:312-338), ready for upload_weights.
// A legacy PRICHS_W file has no indexed parameters and is refused here.
struct Checkpoint {
  uint64_t step = 0;
  float loss = 0.f;
  std::vector<std::vector<float>> params;
};
Checkpoint load_checkpoint(const std::string &path);
// Index of `slot` of block `layer` with E routed experts: 2 + layer * (10 + 3E)
// + slot (model.rs:557-562, 1083-1087).  Throws for a slot past the block.
size_t block_param_index(size_t layer, size_t E, size_t slot);

class GpuModelEngine {
 public:
  // engine.rs:363: one (rows, cols, apply_weight_decay) triple per parameter.
  explicit GpuModelEngine(const std::vector<std::tuple<size_t, size_t, bool>> &param_shapes,
                          const Capacity &cap = Capacity());
  ~GpuModelEngine();
  GpuModelEngine(const GpuModelEngine &) = delete;
  GpuModelEngine &operator=(const GpuModelEngine &) = delete;

  const std::vector<ParamMetadata> &params() const { return meta_; }

  // engine.rs:668-689 / 691-708: one host slice per parameter, reference layout.
  void upload_weights(const std::vector<std::vector<float>> &param_slices);
  void download_weights(std::vector<std::vector<float>> &param_slices) const;

  // engine.rs:757-826: out[m, n] = x[m, k] @ W[param_id] ([k, n]).
  void forward_gemm(size_t param_id, const std::vector<float> &x, std::vector<float> &out,
                    size_t m, size_t k, size_t n);

  // engine.rs:1788-1846: out = (x * rstd) * w per row, rstd = 1/sqrt(mean(x^2) + eps).
  void gpu_rmsnorm_forward(const std::vector<float> &x, size_t param_id, std::vector<float> &out,
                           std::vector<float> &rstd, size_t seq_len, size_t hidden_dim,
                           float eps);

  // engine.rs:1162-1179.
  void upload_rope_cache(const std::vector<float> &cos_cache, const std::vector<float> &sin_cache);

  // engine.rs:1181-1405 (called at model.rs:1101): one sequence's attention
  // sub-layer on host slices.  q/k/v = normed1 [T, d] @ W (f32 MFMA GEMMs),
  // RoPE from the uploaded cache at positions 0..T-1, causal GQA attention with
  // the probabilities kept (prichs_attention_probs_f32), attn_out = concat @ Wo.
  // Returns (q_rope, k_rope, v, probs [H, T, T], concat) like the reference.
  AttentionOut gpu_batched_attention_forward(const std::vector<float> &normed1, size_t q_id,
                                             size_t k_id, size_t v_id, size_t out_id,
                                             std::vector<float> &attn_out, size_t seq_len,
                                             size_t num_heads, size_t num_kv_heads,
                                             size_t head_dim);

  // engine.rs:1917-2051: the shared expert on all rows of normed2, which stays
  // resident for the routed experts; its output starts the MoE accumulator.
  SharedOut gpu_moe_forward_shared(const std::vector<float> &normed2, size_t gate_id,
                                   size_t up_id, size_t down_id, size_t seq_len,
                                   size_t hidden_dim, size_t intermediate_dim);

  // engine.rs:2054-2223: one routed expert on the rows token_indices of the
  // resident normed2; accum[token] += weight * out[row].
  ExpertOut gpu_moe_forward_expert(const std::vector<int32_t> &token_indices,
                                   const std::vector<float> &weights, size_t gate_id,
                                   size_t up_id, size_t down_id, size_t hidden_dim,
                                   size_t intermediate_dim);

  // engine.rs:2226-2239: the accumulated MoE output.
  void gpu_moe_finalize_forward(std::vector<float> &total_out) const;

  // engine.rs:2694-2702.
  void sync_stream() const;

  // ---- Fast path (no reference counterpart): the fused MoE layer on device
  // buffers.  Builds a libprichs_hip MoE engine from registered parameters:
  // router [d, E], the shared expert's (gate, up, down) and each routed
  // expert's, with dtype PRICHS_DTYPE_BF16 or PRICHS_DTYPE_F32.  Returns a
  // layer id.
  size_t create_moe_layer(size_t router_id, const std::vector<float> &router_bias,
                          size_t shared_gate, size_t shared_up, size_t shared_down,
                          const std::vector<std::tuple<size_t, size_t, size_t>> &experts,
                          size_t top_k, int dtype, size_t max_tokens);
  // x [T, d] and out [T, d] are device pointers of the layer's dtype; enqueued
  // on `stream` (a hipStream_t; null = default stream), nothing allocated.
  void gpu_moe_forward(size_t layer_id, const void *x_dev, size_t T, void *out_dev,
                       void *stream = nullptr);
  // The aux-free bias (moe.rs:60) of a layer: set from the host, updated on
  // device from the last forward's routing (moe.rs:228-245 as model.rs:
  // 1541-1547 drives it), read back.
  void set_moe_router_bias(size_t layer_id, const std::vector<float> &router_bias);
  void update_moe_router_bias(size_t layer_id, float gamma, void *stream = nullptr);
  std::vector<float> moe_router_bias(size_t layer_id) const;

 private:
  struct PackedGemm;  // f32 weights packed for prichs_gemm (zero-padded to 16)
  struct MoeLayer {
    prichs_moe_engine *eng = nullptr;
    size_t d = 0, E = 0;
    int dtype = 0;
  };

  void release();  // frees every device buffer and engine (destructor, failed constructor)

  void gemm_dev(size_t param_id, const float *x_dev, size_t ldx, float *out_dev, size_t ldo,
                size_t m);
  const PackedGemm &packed(size_t param_id);
  void check_param(size_t id, const char *who) const;

  std::vector<ParamMetadata> meta_;
  Capacity cap_;
  float *dev_weights_ = nullptr;
  // Workspace (f32): GEMM staging with padded leading dimensions.
  float *dev_act_in_ = nullptr;   // normed2, resident between shared and experts
  float *dev_act_out_ = nullptr;  // forward_gemm / rmsnorm output
  float *dev_x_ = nullptr;        // gathered expert rows
  float *dev_gate_ = nullptr, *dev_up_ = nullptr, *dev_act_ = nullptr;
  float *dev_out_ = nullptr;      // expert output rows
  float *dev_moe_out_ = nullptr;  // MoE accumulator
  float *dev_rstd_ = nullptr;
  float *dev_cos_ = nullptr, *dev_sin_ = nullptr;
  size_t rope_len_ = 0;  // entries of the last uploaded cos / sin cache
  // attention scratch (q, k, v, concat, probabilities), allocated on first use
  float *dev_q_ = nullptr, *dev_k_ = nullptr, *dev_v_ = nullptr, *dev_cat_ = nullptr;
  float *dev_probs_ = nullptr;
  int32_t *dev_idx_ = nullptr;
  float *dev_w_ = nullptr;
  size_t moe_rows_ = 0, moe_ld_ = 0, moe_d_ = 0;  // layout of the accumulator
  size_t act_in_ld_ = 0;                         // leading dimension of normed2
  std::vector<PackedGemm *> packed_;
  std::vector<MoeLayer> layers_;
};

// GpuWorkspace (crates/prichs-cuda/src/cublas.rs:46-268) over
// prichs_gpu_workspace_*: device slabs for A, B and C (sizes in bytes; 0 = the
// reference's 16 MB / 32 MB / 16 MB) and the three host-slice GEMMs, each
// H2D, GEMM, D2H and a device synchronisation.  Slices must hold at least the
// elements (m, k, n) name; an operand larger than its slab throws the
// reference's "exceed preallocated GPU workspace slabs" error.  dw / dx are
// overwritten, like the reference's GPU path.
class GpuWorkspace {
 public:
  explicit GpuWorkspace(size_t a_bytes = 0, size_t b_bytes = 0, size_t c_bytes = 0);
  ~GpuWorkspace();
  GpuWorkspace(const GpuWorkspace &) = delete;
  GpuWorkspace &operator=(const GpuWorkspace &) = delete;

  // cublas.rs:117-166: c [m, n] = a [m, k] b [k, n].
  void matmul(const std::vector<float> &a, const std::vector<float> &b, std::vector<float> &c,
              size_t m, size_t k, size_t n) const;
  // cublas.rs:170-219: dw [k, n] = a [m, k]^T b [m, n].
  void matmul_at_b(const std::vector<float> &a, const std::vector<float> &b,
                   std::vector<float> &dw, size_t m, size_t k, size_t n) const;
  // cublas.rs:221-268: dx [m, n] = dy [m, k] w [n, k]^T.
  void matmul_a_bt(const std::vector<float> &dy, const std::vector<float> &w,
                   std::vector<float> &dx, size_t m, size_t k, size_t n) const;

 private:
  friend GpuWorkspace *get_gpu_workspace();
  explicit GpuWorkspace(prichs_gpu_workspace *borrowed);  // the process-wide one
  prichs_gpu_workspace *ws_ = nullptr;
  bool owned_ = true;
};

// get_gpu_workspace (cublas.rs:283-300): the process-wide workspace, or null
// when it could not be created (no device).
GpuWorkspace *get_gpu_workspace();
// matmul_gpu / matmul_at_b_gpu / matmul_a_bt_gpu (cublas.rs:302-327): the
// methods above on the process-wide workspace, serialised by one mutex;
// without a workspace they throw "GPU workspace unavailable".
void matmul_gpu(const std::vector<float> &a, const std::vector<float> &b, std::vector<float> &c,
                size_t m, size_t k, size_t n);
void matmul_at_b_gpu(const std::vector<float> &a, const std::vector<float> &b,
                     std::vector<float> &dw, size_t m, size_t k, size_t n);
void matmul_a_bt_gpu(const std::vector<float> &dy, const std::vector<float> &w,
                     std::vector<float> &dx, size_t m, size_t k, size_t n);

}  // namespace prichs_host
