// noalloc.hip -- the MoE layer forward without any device allocation.
//
// prichs_moe_forward_noalloc runs the computation of prichs_moe_engine_forward
// (router + top-k, permutation, grouped gate/up + SwiGLU, grouped down,
// combine; the same kernels in the same order) for callers that cannot call
// hipMalloc: code under HIP graph capture, tight serving loops, harnesses
// that forbid allocation.  The caller passes x, the layer's weights (already
// on the device) and out; every intermediate lives in `scratch`, a
// file-scope device array of PRICHS_NOALLOC_SCRATCH_BYTES that each GPU holds
// from the library's load until the process ends.  Calls on one GPU share
// it and it keeps the last call's contents: every kernel writes each
// intermediate it reads later, so nothing needs clearing, and two calls that
// overlap on one GPU (two streams, two threads) race on it.
#include <mutex>

#include "common.hpp"

static __device__ __align__(256) unsigned char scratch[PRICHS_NOALLOC_SCRATCH_BYTES];

namespace prichs {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// The device address of this device's copy of `scratch`, looked up once per
// device (with that device current) and kept.  In host code `scratch` names
// a host-side stand-in, never the device memory: only this address may be
// handed to kernels or copies.
int scratch_address(void **out) {
  int dev = -1;
  PRICHS_HIP_TRY(hipGetDevice(&dev), "moe_forward_noalloc: no HIP device");
  if (dev < 0 || dev >= kMaxDevices)
    return fail(PRICHS_ERR_UNSUPPORTED, "moe_forward_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(PRICHS_ERR_HIP, "moe_forward_noalloc: hipGetSymbolAddress(scratch): %s",
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return PRICHS_OK;
}

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

extern "C" int prichs_moe_forward_noalloc(const void *x, size_t T, size_t d, size_t f, size_t E,
                                          size_t k, size_t n_shared, int dtype,
                                          const float *w_router, const float *router_bias,
                                          const void *w_gate_up, const void *w_down,
                                          const float *concept_bias, size_t n_concept, void *out,
                                          int out_dtype, void *stream) {
  PRICHS_REQUIRE(dtype_ok(dtype) && dtype_ok(out_dtype),
                 "moe_forward_noalloc: bad dtype %d / out dtype %d", dtype, out_dtype);
  PRICHS_REQUIRE(E >= 1 && E <= PRICHS_MAX_EXPERTS, "moe_forward_noalloc: E=%zu outside [1, %d]",
                 E, PRICHS_MAX_EXPERTS);
  PRICHS_REQUIRE(k >= 1 && k <= E && k <= PRICHS_MAX_TOPK,
                 "moe_forward_noalloc: k=%zu invalid for E=%zu", k, E);
  PRICHS_REQUIRE(n_shared <= 1, "moe_forward_noalloc: n_shared=%zu (0 or 1 supported)", n_shared);
  PRICHS_REQUIRE(concept_bias != nullptr || n_concept == 0,
                 "moe_forward_noalloc: concept_bias is NULL but n_concept=%zu", n_concept);
  PRICHS_REQUIRE(d >= 1 && f >= 1 && d <= ((size_t)1 << 20) && f <= ((size_t)1 << 20) &&
                     T <= (size_t)INT32_MAX / (k + 1),
                 "moe_forward_noalloc: T=%zu, d=%zu, f=%zu out of range", T, d, f);
  if (T == 0) return PRICHS_OK;
  PRICHS_REQUIRE(x && w_router && router_bias && w_gate_up && w_down && out,
                 "moe_forward_noalloc: null pointer argument");

  // The engine's workspace layout for T tokens, carved from the scratch.
  const size_t es = dtype_size(dtype);
  const size_t G = E + n_shared;
  const size_t rows = T * k + n_shared * T;
  const size_t nb = prichs_router_num_blocks(T, E);
  Carve c;
  const size_t o_logits = c.take(sizeof(float) * T * E);
  const size_t o_idx = c.take(sizeof(int32_t) * T * k);
  const size_t o_w = c.take(sizeof(float) * T * k);
  const size_t o_bc = c.take(sizeof(int32_t) * nb * E);
  const size_t o_off = c.take(sizeof(int32_t) * (E + 2));
  const size_t o_rt = c.take(sizeof(int32_t) * (T * k + T));
  const size_t o_rw = c.take(sizeof(float) * T * k);
  const size_t o_tr = c.take(sizeof(int32_t) * T * k);
  const size_t o_act = c.take(es * rows * f);
  const size_t o_y = c.take(es * rows * d);
  if (c.off > (size_t)PRICHS_NOALLOC_SCRATCH_BYTES)
    return fail(PRICHS_ERR_CAPACITY,
                "moe_forward_noalloc: T=%zu (d=%zu, f=%zu, E=%zu, k=%zu) needs %zu bytes of "
                "scratch; it holds %zu",
                T, d, f, E, k, c.off, (size_t)PRICHS_NOALLOC_SCRATCH_BYTES);

  void *base_v = nullptr;
  if (int rc = scratch_address(&base_v)) return rc;
  char *base = static_cast<char *>(base_v);
  float *logits = reinterpret_cast<float *>(base + o_logits);
  int32_t *topk_idx = reinterpret_cast<int32_t *>(base + o_idx);
  float *topk_w = reinterpret_cast<float *>(base + o_w);
  int32_t *block_counts = reinterpret_cast<int32_t *>(base + o_bc);
  int32_t *offsets = reinterpret_cast<int32_t *>(base + o_off);
  int32_t *row_token = reinterpret_cast<int32_t *>(base + o_rt);
  float *row_weight = reinterpret_cast<float *>(base + o_rw);
  int32_t *token_row = reinterpret_cast<int32_t *>(base + o_tr);
  void *act = base + o_act;
  void *y = base + o_y;

  int rc = router_topk_permute(x, dtype, w_router, router_bias, concept_bias, n_concept, T, d, E,
                               k, logits, topk_idx, topk_w, block_counts, offsets, row_token,
                               row_weight, token_row, stream);
  if (rc) return rc;
  // No group holds more than T rows (a token picks an expert at most once).
  rc = grouped_gate_up_swiglu_rows(x, row_token, offsets, G, rows, T, w_gate_up, d, f, dtype, act,
                                   stream, nullptr);
  if (rc) return rc;
  rc = grouped_down_rows(act, offsets, G, rows, T, w_down, d, f, dtype, y, stream);
  if (rc) return rc;
  return prichs_moe_combine(y, dtype, topk_idx, topk_w, token_row, T, d, k, (int)n_shared, out,
                            out_dtype, stream);
}
