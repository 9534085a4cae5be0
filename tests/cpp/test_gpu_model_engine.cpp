// test_gpu_model_engine.cpp -- tests of the C++ GpuModelEngine mirror
// (prichs_amd/host/gpu_model_engine.hpp), written like the reference's own
// engine tests (crates/prichs-cuda/src/engine.rs:2876-3182): same data, same
// calls, same tolerances, plus checks of the values the reference only prints.
//
// usage: test_gpu_model_engine                run the GPU tests
//        test_gpu_model_engine --no-gpu       only the host tests: the
//                                              checkpoint loader, and engine
//                                              creation without a device
//                                              failing cleanly
//        test_gpu_model_engine FIXTURE_DIR    also the config-1 parity test on
//                                              oracle fixtures (see
//                                              tests/test_host_cpp.py)
// Exit status 0 when every test passed.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <functional>
#include <map>
#include <sstream>
#include <string>
#include <vector>

#include <unistd.h>

#include "gpu_model_engine.hpp"
#include "prichs_hip.h"

using prichs_host::Error;
using prichs_host::GpuModelEngine;

namespace {

int g_failed = 0;

#define CHECK(cond, ...)                                  \
  do {                                                    \
    if (!(cond)) {                                        \
      std::printf("    FAIL %s:%d: ", __FILE__, __LINE__); \
      std::printf(__VA_ARGS__);                           \
      std::printf("\n");                                  \
      throw std::runtime_error("check failed");           \
    }                                                     \
  } while (0)

void run(const char *name, const std::function<void()> &fn) {
  std::printf("[ RUN  ] %s\n", name);
  std::fflush(stdout);
  try {
    fn();
    std::printf("[  OK  ] %s\n", name);
  } catch (const std::exception &e) {
    ++g_failed;
    std::printf("[ FAIL ] %s: %s\n", name, e.what());
  }
  std::fflush(stdout);
}

// Runs fn, which must throw prichs_host::Error whose message contains `what`.
void expect_error(const std::function<void()> &fn, const char *what) {
  try {
    fn();
  } catch (const Error &e) {
    CHECK(std::strstr(e.what(), what) != nullptr, "error '%s' lacks '%s'", e.what(), what);
    return;
  }
  CHECK(false, "no error raised (expected '%s')", what);
}

float silu(float x) { return x / (1.0f + std::exp(-x)); }

double rel_err(const std::vector<float> &a, const std::vector<float> &b) {
  double num = 0, den = 0;
  for (size_t i = 0; i < a.size(); ++i) {
    num = std::max(num, (double)std::fabs(a[i] - b[i]));
    den = std::max(den, (double)std::fabs(b[i]));
  }
  return den > 0 ? num / den : num;
}

// engine.rs:2876-2908 (forward half of test_persistent_vram_gemm_correctness).
void test_persistent_vram_gemm_correctness() {
  std::vector<std::tuple<size_t, size_t, bool>> shapes{{4, 3, true}};
  GpuModelEngine engine(shapes);
  const std::vector<float> w_host{1.0f, 2.0f, 3.0f, 4.0f, 5.0f, 6.0f,
                                  7.0f, 8.0f, 9.0f, 10.0f, 11.0f, 12.0f};
  engine.upload_weights({w_host});
  const std::vector<float> x_host{1.0f, 0.5f, 0.2f, 0.1f, 2.0f, 1.0f, 0.0f, -1.0f};
  std::vector<float> out_gpu(2 * 3, 0.0f);
  engine.forward_gemm(0, x_host, out_gpu, 2, 4, 3);
  for (int i = 0; i < 2; ++i)
    for (int j = 0; j < 3; ++j) {
      float sum = 0.0f;
      for (int k = 0; k < 4; ++k) sum += x_host[i * 4 + k] * w_host[k * 3 + j];
      const float diff = std::fabs(out_gpu[i * 3 + j] - sum);
      CHECK(diff < 1e-4f, "Forward mismatch at %d: gpu %g vs cpu %g", i * 3 + j,
            out_gpu[i * 3 + j], sum);
    }
  std::vector<std::vector<float>> back(1);
  engine.download_weights(back);
  CHECK(back[0] == w_host, "download_weights returned different weights");
}

// engine.rs:2877-2936 through prichs-core's GPU dispatch target: forward
// x W with matmul_gpu, backward-data dY W^T with matmul_a_bt_gpu and
// backward-weight x^T dY with matmul_at_b_gpu (cublas.rs:302-327), against
// the CPU triple loops within 1e-4; the workspace has the reference's slabs
// and refuses an operand larger than its slab.
void test_matmul_gpu_family() {
  const std::vector<float> w{1.0f, 2.0f, 3.0f, 4.0f, 5.0f, 6.0f,
                             7.0f, 8.0f, 9.0f, 10.0f, 11.0f, 12.0f};
  const std::vector<float> x{1.0f, 0.5f, 0.2f, 0.1f, 2.0f, 1.0f, 0.0f, -1.0f};
  const std::vector<float> dy{0.5f, -0.5f, 1.0f, 1.0f, 2.0f, -1.0f};
  std::vector<float> out(6), dx(8), dw(12, 7.0f);
  prichs_host::matmul_gpu(x, w, out, 2, 4, 3);
  prichs_host::matmul_a_bt_gpu(dy, w, dx, 2, 3, 4);
  prichs_host::matmul_at_b_gpu(x, dy, dw, 2, 4, 3);
  for (int i = 0; i < 2; ++i)
    for (int j = 0; j < 3; ++j) {
      float sum = 0.0f;
      for (int k = 0; k < 4; ++k) sum += x[i * 4 + k] * w[k * 3 + j];
      CHECK(std::fabs(out[i * 3 + j] - sum) < 1e-4f, "matmul_gpu mismatch at %d", i * 3 + j);
    }
  for (int i = 0; i < 2; ++i)
    for (int k = 0; k < 4; ++k) {
      float sum = 0.0f;
      for (int j = 0; j < 3; ++j) sum += dy[i * 3 + j] * w[k * 3 + j];
      CHECK(std::fabs(dx[i * 4 + k] - sum) < 1e-4f, "matmul_a_bt_gpu mismatch at %d", i * 4 + k);
    }
  for (int k = 0; k < 4; ++k)
    for (int j = 0; j < 3; ++j) {
      float sum = 0.0f;
      for (int i = 0; i < 2; ++i) sum += x[i * 4 + k] * dy[i * 3 + j];
      CHECK(std::fabs(dw[k * 3 + j] - sum) < 1e-4f, "matmul_at_b_gpu mismatch at %d", k * 3 + j);
    }
  prichs_host::GpuWorkspace *ws = prichs_host::get_gpu_workspace();
  CHECK(ws != nullptr, "no process-wide workspace");
  CHECK(prichs_host::get_gpu_workspace() == ws, "the process-wide workspace changed");
  // slab A holds 4 Mi floats (16 MB): 4097 x 1024 does not fit
  std::vector<float> big(4097 * 1024, 1.0f), bb(1024, 1.0f), cc(4097, 0.0f);
  expect_error([&] { ws->matmul(big, bb, cc, 4097, 1024, 1); }, "exceed preallocated");
  prichs_host::GpuWorkspace own(4097 * 1024 * 4, 0, 0);
  own.matmul(big, bb, cc, 4097, 1024, 1);
  CHECK(cc[0] == 1024.0f && cc[4096] == 1024.0f, "sums of 1024 ones: %g %g", cc[0], cc[4096]);
  expect_error([&] { own.matmul(bb, bb, cc, 4097, 1024, 1); }, "elements");
}

// engine.rs:2948-3005 (test_gpu_batched_attention_execution): the reference's
// data, its length / row-sum / causal checks, plus the closed form that data
// has (every projection 0.4, uniform causal rows, attn_out 8 * 0.4 * 0.1).
void test_gpu_batched_attention_execution() {
  const size_t T = 4, H = 2, KV = 1, hd = 4, hidden = H * hd, kvd = KV * hd;
  GpuModelEngine eng({{hidden, hidden, true}, {hidden, kvd, true}, {hidden, kvd, true},
                      {hidden, hidden, true}});
  eng.upload_weights({std::vector<float>(hidden * hidden, 0.1f),
                      std::vector<float>(hidden * kvd, 0.1f),
                      std::vector<float>(hidden * kvd, 0.1f),
                      std::vector<float>(hidden * hidden, 0.1f)});
  eng.upload_rope_cache(std::vector<float>(T * (hd / 2), 1.0f),
                        std::vector<float>(T * (hd / 2), 0.0f));
  const std::vector<float> normed1(T * hidden, 0.5f);
  std::vector<float> attn_out(T * hidden, 0.0f);
  auto [q, k, v, probs, concat] =
      eng.gpu_batched_attention_forward(normed1, 0, 1, 2, 3, attn_out, T, H, KV, hd);
  CHECK(q.size() == T * hidden && k.size() == T * kvd && v.size() == T * kvd, "lengths");
  CHECK(probs.size() == H * T * T && concat.size() == T * hidden, "lengths");
  for (size_t h = 0; h < H; ++h)
    for (size_t i = 0; i < T; ++i) {
      const float *row = &probs[h * T * T + i * T];
      float sum = 0.0f;
      for (size_t j = 0; j < T; ++j) sum += row[j];
      CHECK(std::fabs(sum - 1.0f) < 1e-4f, "softmax sum %g at h=%zu i=%zu", sum, h, i);
      for (size_t j = i + 1; j < T; ++j) CHECK(row[j] == 0.0f, "causal violation %zu %zu", i, j);
      for (size_t j = 0; j <= i; ++j)
        CHECK(std::fabs(row[j] - 1.0f / (i + 1)) < 1e-5f, "uniform row %zu: %g", i, row[j]);
    }
  for (float x : q) CHECK(std::fabs(x - 0.4f) < 1e-5f, "q %g", x);
  for (float x : k) CHECK(std::fabs(x - 0.4f) < 1e-5f, "k %g", x);
  for (float x : v) CHECK(std::fabs(x - 0.4f) < 1e-5f, "v %g", x);
  for (float x : concat) CHECK(std::fabs(x - 0.4f) < 1e-5f, "concat %g", x);
  for (float x : attn_out) CHECK(std::fabs(x - 0.32f) < 1e-5f, "attn_out %g", x);
}

// The same method on random weights and a real RoPE cache against a
// double-precision host computation of the textbook causal GQA attention.
void test_gpu_batched_attention_random() {
  const size_t T = 37, H = 4, KV = 2, hd = 16, hidden = H * hd, kvd = KV * hd, half = hd / 2;
  unsigned seed = 12345;
  auto rnd = [&] {
    seed = seed * 1664525u + 1013904223u;
    return ((seed >> 8) * (1.0f / 16777216.0f)) - 0.5f;
  };
  auto fill = [&](size_t n, float scale) {
    std::vector<float> w(n);
    for (auto &x : w) x = scale * rnd();
    return w;
  };
  std::vector<std::vector<float>> w{fill(hidden * hidden, 0.3f), fill(hidden * kvd, 0.3f),
                                    fill(hidden * kvd, 0.3f), fill(hidden * hidden, 0.3f)};
  GpuModelEngine eng({{hidden, hidden, true}, {hidden, kvd, true}, {hidden, kvd, true},
                      {hidden, hidden, true}});
  eng.upload_weights(w);
  std::vector<float> cosc(T * half), sinc(T * half);
  for (size_t t = 0; t < T; ++t)
    for (size_t i = 0; i < half; ++i) {
      const double ang = t * std::pow(10000.0, -2.0 * i / hd);
      cosc[t * half + i] = (float)std::cos(ang);
      sinc[t * half + i] = (float)std::sin(ang);
    }
  std::vector<float> normed1 = fill(T * hidden, 2.0f), attn_out(T * hidden, 0.0f);
  // A cache shorter than seq_len is refused before any launch.
  eng.upload_rope_cache(std::vector<float>(half), std::vector<float>(half));
  expect_error([&] {
    eng.gpu_batched_attention_forward(normed1, 0, 1, 2, 3, attn_out, T, H, KV, hd);
  }, "RoPE cache");
  expect_error([&] {
    std::vector<float> short_out(5);
    eng.gpu_batched_attention_forward(normed1, 0, 1, 2, 3, short_out, T, H, KV, hd);
  }, "attn_out length mismatch");
  eng.upload_rope_cache(cosc, sinc);
  auto [q, k, v, probs, concat] =
      eng.gpu_batched_attention_forward(normed1, 0, 1, 2, 3, attn_out, T, H, KV, hd);
  auto proj = [&](const std::vector<float> &x, const std::vector<float> &wm, size_t n) {
    std::vector<double> y(T * n, 0.0);
    for (size_t t = 0; t < T; ++t)
      for (size_t c = 0; c < hidden; ++c)
        for (size_t j = 0; j < n; ++j) y[t * n + j] += (double)x[t * hidden + c] * wm[c * n + j];
    return y;
  };
  auto rope = [&](std::vector<double> &y, size_t heads) {
    for (size_t t = 0; t < T; ++t)
      for (size_t h = 0; h < heads; ++h)
        for (size_t i = 0; i < half; ++i) {
          double *p = &y[t * heads * hd + h * hd + 2 * i];
          const double c = cosc[t * half + i], s = sinc[t * half + i];
          const double a = p[0], b = p[1];
          p[0] = a * c - b * s;
          p[1] = a * s + b * c;
        }
  };
  std::vector<double> rq = proj(normed1, w[0], hidden), rk = proj(normed1, w[1], kvd),
                      rv = proj(normed1, w[2], kvd);
  rope(rq, H);
  rope(rk, KV);
  std::vector<double> rp(H * T * T, 0.0), rc(T * hidden, 0.0);
  for (size_t h = 0; h < H; ++h) {
    const size_t g = h / (H / KV);
    for (size_t i = 0; i < T; ++i) {
      double m = -1e300, sum = 0.0;
      std::vector<double> s(i + 1);
      for (size_t j = 0; j <= i; ++j) {
        double d = 0.0;
        for (size_t c = 0; c < hd; ++c) d += rq[i * hidden + h * hd + c] * rk[j * kvd + g * hd + c];
        s[j] = d / std::sqrt((double)hd);
        m = std::max(m, s[j]);
      }
      for (size_t j = 0; j <= i; ++j) sum += (s[j] = std::exp(s[j] - m));
      for (size_t j = 0; j <= i; ++j) {
        rp[h * T * T + i * T + j] = s[j] / sum;
        for (size_t c = 0; c < hd; ++c)
          rc[i * hidden + h * hd + c] += s[j] / sum * rv[j * kvd + g * hd + c];
      }
    }
  }
  std::vector<double> ro(T * hidden, 0.0);
  for (size_t t = 0; t < T; ++t)
    for (size_t c = 0; c < hidden; ++c)
      for (size_t j = 0; j < hidden; ++j) ro[t * hidden + j] += rc[t * hidden + c] * w[3][c * hidden + j];
  auto close = [&](const std::vector<float> &got, const std::vector<double> &want, const char *what) {
    double err = 0.0, mag = 0.0;
    for (size_t i = 0; i < want.size(); ++i) {
      err = std::max(err, std::fabs(got[i] - want[i]));
      mag = std::max(mag, std::fabs(want[i]));
    }
    CHECK(err <= 1e-4 * std::max(mag, 1.0), "%s: max error %g (magnitude %g)", what, err, mag);
  };
  close(q, rq, "q_rope");
  close(k, rk, "k_rope");
  close(v, rv, "v");
  close(probs, rp, "probs");
  close(concat, rc, "concat");
  close(attn_out, ro, "attn_out");
}

// engine.rs:3032-3053 (forward half of test_gpu_rmsnorm_correctness).
void test_gpu_rmsnorm_correctness() {
  const size_t seq_len = 2, hidden_dim = 4;
  GpuModelEngine engine({{1, hidden_dim, false}});
  engine.upload_weights({{1.0f, 1.0f, 1.0f, 1.0f}});
  const std::vector<float> x{1.0f, 2.0f, 3.0f, 4.0f, 2.0f, 2.0f, 2.0f, 2.0f};
  std::vector<float> out(seq_len * hidden_dim, 0.0f), rstd(seq_len, 0.0f);
  engine.gpu_rmsnorm_forward(x, 0, out, rstd, seq_len, hidden_dim, 1e-5f);
  // Row 1: mean_sq = 4, rstd = 1/sqrt(4 + 1e-5), out = 2 * rstd ~ 1.0.
  for (size_t d = 4; d < 8; ++d) CHECK(std::fabs(out[d] - 1.0f) < 1e-4f, "Expected 1.0, got %g", out[d]);
  // Row 0 in closed form: mean_sq = 7.5.
  const float r0 = 1.0f / std::sqrt(7.5f + 1e-5f);
  CHECK(std::fabs(rstd[0] - r0) < 1e-6f, "rstd[0] %g vs %g", rstd[0], r0);
  for (size_t d = 0; d < 4; ++d)
    CHECK(std::fabs(out[d] - x[d] * r0) < 1e-5f, "row 0 col %zu: %g vs %g", d, out[d], x[d] * r0);
}

// engine.rs:3067-3130 (forward half of test_gpu_moe_forward_backward), with
// the closed-form value of the output the reference only checks for non-zero.
void test_gpu_moe_forward() {
  const size_t seq_len = 2, hidden_dim = 4, intermediate_dim = 8, num_experts = 2;
  const size_t d = hidden_dim, f = intermediate_dim;
  GpuModelEngine engine({
      {d, f, true}, {d, f, true}, {f, d, true},   // shared gate / up / down
      {d, f, true}, {d, f, true}, {f, d, true},   // expert 0
      {d, f, true}, {d, f, true}, {f, d, true},   // expert 1
      {d, num_experts, true},                     // router
  });
  const std::vector<float> w_gate(d * f, 0.1f), w_up(d * f, 0.1f), w_down(f * d, 0.1f),
      w_router(d * num_experts, 0.1f);
  engine.upload_weights(
      {w_gate, w_up, w_down, w_gate, w_up, w_down, w_gate, w_up, w_down, w_router});
  const std::vector<float> normed2(seq_len * d, 0.5f);

  auto [s_gate, s_up, s_act, s_out] =
      engine.gpu_moe_forward_shared(normed2, 0, 1, 2, seq_len, hidden_dim, intermediate_dim);
  CHECK(s_out.size() == seq_len * hidden_dim, "shared out has %zu elements", s_out.size());
  // gate = up = 4 * 0.5 * 0.1 = 0.2; act = silu(0.2) * 0.2; out = 8 * act * 0.1.
  const float g = 0.2f, a = silu(g) * g, o = 0.8f * a;
  for (float v : s_gate) CHECK(std::fabs(v - g) < 1e-6f, "gate %g vs %g", v, g);
  for (float v : s_act) CHECK(std::fabs(v - a) < 1e-6f, "act %g vs %g", v, a);
  for (float v : s_out) CHECK(std::fabs(v - o) < 1e-6f, "shared out %g vs %g", v, o);

  const std::vector<int32_t> token_indices{0, 1};
  const std::vector<float> weights{0.5f, 0.5f};
  auto [e0_x, e0_gate, e0_up, e0_act, e0_out] =
      engine.gpu_moe_forward_expert(token_indices, weights, 3, 4, 5, hidden_dim, intermediate_dim);
  CHECK(e0_out.size() == seq_len * hidden_dim, "expert out has %zu elements", e0_out.size());
  CHECK(e0_x == normed2, "gathered rows differ from normed2");

  std::vector<float> total_moe_out(seq_len * hidden_dim, 0.0f);
  engine.gpu_moe_finalize_forward(total_moe_out);
  bool has_nonzero = false;
  for (float v : total_moe_out) has_nonzero |= std::fabs(v) > 1e-6f;
  CHECK(has_nonzero, "MoE forward output must be non-zero");
  // shared + 0.5 * expert0 (same weights) = 1.5 * o.
  for (float v : total_moe_out) CHECK(std::fabs(v - 1.5f * o) < 1e-6f, "total %g vs %g", v, 1.5f * o);

  // An empty expert returns empty results and leaves the accumulator alone.
  auto empty = engine.gpu_moe_forward_expert({}, {}, 6, 7, 8, hidden_dim, intermediate_dim);
  CHECK(std::get<4>(empty).empty(), "empty expert returned rows");
}

// The reference's bail! paths (engine.rs:767-777, 1788-1800, 1934-1936) and
// this mirror's stricter checks: each raises an Error, nothing crashes.
void test_error_paths() {
  GpuModelEngine engine({{4, 3, true}, {1, 4, false}},
                        prichs_host::Capacity{64, 64, 64, 64, 8});
  expect_error([&] { engine.upload_weights({{1.0f}}); }, "param_slices count");
  expect_error([&] { engine.upload_weights({{1.0f}, {1.0f}}); }, "length mismatch");
  engine.upload_weights({std::vector<float>(12, 1.0f), std::vector<float>(4, 1.0f)});
  std::vector<float> out(6), x(8, 1.0f);
  expect_error([&] { engine.forward_gemm(0, x, out, 2, 3, 4); }, "shape mismatch");
  expect_error([&] { engine.forward_gemm(7, x, out, 2, 4, 3); }, "out of range");
  std::vector<float> big(64 * 4, 1.0f), bigout(64 * 3);
  expect_error([&] { engine.forward_gemm(0, big, bigout, 64, 4, 3); }, "exceed");
  std::vector<float> r(2);
  expect_error([&] { engine.gpu_rmsnorm_forward(x, 0, out, r, 2, 4, 1e-5f); }, "len mismatch");
  expect_error([&] { engine.gpu_moe_forward_expert({0}, {1.0f}, 0, 0, 0, 4, 3); }, "MoE expert weights");
  expect_error([&] { engine.upload_rope_cache({1.0f}, {1.0f, 2.0f}); }, "equal length");
  expect_error([&] { engine.gpu_moe_forward(0, nullptr, 1, nullptr); }, "no MoE layer");
}

// ---- Config-1 parity on oracle fixtures -----------------------------------
struct Fixture {
  std::map<std::string, std::vector<float>> f32;
  std::map<std::string, std::vector<int32_t>> i32;
  std::map<std::string, size_t> scalar;
};

Fixture load_fixture(const std::string &dir) {
  Fixture fx;
  std::ifstream man(dir + "/manifest.txt");
  CHECK(man.good(), "cannot open %s/manifest.txt", dir.c_str());
  std::string line;
  while (std::getline(man, line)) {
    std::istringstream ls(line);
    std::string kind, name;
    size_t n = 0;
    ls >> kind >> name >> n;
    if (kind == "scalar") {
      fx.scalar[name] = n;
      continue;
    }
    std::ifstream in(dir + "/" + name + ".bin", std::ios::binary);
    CHECK(in.good(), "cannot open %s.bin", name.c_str());
    if (kind == "f32") {
      fx.f32[name].resize(n);
      in.read(reinterpret_cast<char *>(fx.f32[name].data()), n * 4);
    } else {
      fx.i32[name].resize(n);
      in.read(reinterpret_cast<char *>(fx.i32[name].data()), n * 4);
    }
    CHECK(in.good(), "short read of %s", name.c_str());
  }
  return fx;
}

// The reference's per-layer MoE sequence (model.rs:1125-1177) on the mirror:
// router logits through forward_gemm, the shared expert, each routed expert
// on the oracle's token lists, finalize; then the fused device path.
void test_moe_config1_parity(const std::string &dir) {
  Fixture fx = load_fixture(dir);
  const size_t T = fx.scalar.at("T"), d = fx.scalar.at("d"), f = fx.scalar.at("f"),
               E = fx.scalar.at("E"), k = fx.scalar.at("k");
  std::vector<std::tuple<size_t, size_t, bool>> shapes;
  std::vector<std::vector<float>> weights;
  for (size_t j = 0; j <= E; ++j) {  // expert j: 0 = shared, 1.. = routed 0..E-1
    shapes.push_back({d, f, true});
    shapes.push_back({d, f, true});
    shapes.push_back({f, d, true});
    weights.push_back(fx.f32.at("gate" + std::to_string(j)));
    weights.push_back(fx.f32.at("up" + std::to_string(j)));
    weights.push_back(fx.f32.at("down" + std::to_string(j)));
  }
  const size_t router_id = shapes.size();
  shapes.push_back({d, E, true});
  weights.push_back(fx.f32.at("w_router"));
  GpuModelEngine engine(shapes);
  engine.upload_weights(weights);
  const std::vector<float> &x = fx.f32.at("x");

  std::vector<float> logits(T * E);
  engine.forward_gemm(router_id, x, logits, T, d, E);
  const double e_log = rel_err(logits, fx.f32.at("logits"));
  std::printf("    router logits rel err %.2e\n", e_log);
  CHECK(e_log <= 1e-5, "router logits rel err %.3e", e_log);

  engine.gpu_moe_forward_shared(x, 0, 1, 2, T, d, f);
  const std::vector<int32_t> &off = fx.i32.at("offsets"), &rt = fx.i32.at("row_token");
  const std::vector<float> &rw = fx.f32.at("row_weight");
  for (size_t e = 0; e < E; ++e) {
    std::vector<int32_t> idx(rt.begin() + off[e], rt.begin() + off[e + 1]);
    std::vector<float> w(rw.begin() + off[e], rw.begin() + off[e + 1]);
    const size_t base = 3 * (e + 1);
    engine.gpu_moe_forward_expert(idx, w, base, base + 1, base + 2, d, f);
  }
  std::vector<float> out(T * d);
  engine.gpu_moe_finalize_forward(out);
  const double e_out = rel_err(out, fx.f32.at("out"));
  std::printf("    stage-by-stage MoE output rel err %.2e (k = %zu)\n", e_out, k);
  CHECK(e_out <= 1e-4, "MoE output rel err %.3e > 1e-4", e_out);

  // The fused path: router, top-k, permutation and both grouped GEMMs on device.
  std::vector<std::tuple<size_t, size_t, size_t>> experts;
  for (size_t e = 0; e < E; ++e) experts.push_back({3 * (e + 1), 3 * (e + 1) + 1, 3 * (e + 1) + 2});
  const size_t layer = engine.create_moe_layer(router_id, fx.f32.at("router_bias"), 0, 1, 2,
                                               experts, k, PRICHS_DTYPE_F32, T);
  float *x_dev = nullptr, *o_dev = nullptr;
  CHECK(hipMalloc((void **)&x_dev, T * d * 4) == hipSuccess, "hipMalloc");
  CHECK(hipMalloc((void **)&o_dev, T * d * 4) == hipSuccess, "hipMalloc");
  CHECK(hipMemcpy(x_dev, x.data(), T * d * 4, hipMemcpyHostToDevice) == hipSuccess, "H2D");
  engine.gpu_moe_forward(layer, x_dev, T, o_dev);
  engine.sync_stream();
  std::vector<float> fused(T * d);
  CHECK(hipMemcpy(fused.data(), o_dev, T * d * 4, hipMemcpyDeviceToHost) == hipSuccess, "D2H");
  (void)hipFree(x_dev);
  (void)hipFree(o_dev);
  const double e_fused = rel_err(fused, fx.f32.at("out"));
  std::printf("    fused MoE output rel err %.2e\n", e_fused);
  CHECK(e_fused <= 1e-4, "fused MoE output rel err %.3e > 1e-4", e_fused);

  // The aux-loss-free update of the training step (model.rs:1541-1547,
  // moe.rs:228-245) on device, against the same f32 steps on the host.
  engine.update_moe_router_bias(layer, 0.001f);
  const std::vector<float> b = engine.moe_router_bias(layer);
  const std::vector<float> &b0 = fx.f32.at("router_bias");
  for (size_t e = 0; e < E; ++e) {
    const float target = (float)k / (float)E;
    const float actual = (float)(off[e + 1] - off[e]) / (float)T;
    const float diff = target - actual;
    const float step = 0.001f * diff;
    const float want = b0[e] + step;
    CHECK(b[e] == want, "bias[%zu] %.9g vs %.9g", e, b[e], want);
  }
}

}  // namespace

// Model::save_checkpoint's layout (model.rs:1648-1670), written here byte by
// byte; load_checkpoint must return every tensor bit for bit, and the block
// index map must name the right tensors.
void test_load_checkpoint() {
  const std::string path = "/tmp/prichs_cpp_ckpt_" + std::to_string(::getpid()) + ".prichs";
  const size_t E = 2, d = 3;
  std::vector<std::vector<float>> params;
  params.push_back({0.5f, -1.f});  // wte
  params.push_back({1.f, 1.f, 1.f});  // final_norm
  for (size_t s = 0; s < 10 + 3 * E; ++s) {  // one block, tensor s filled with 100 + s
    std::vector<float> t(d + s);
    for (size_t i = 0; i < t.size(); ++i) t[i] = 100.f + (float)s + 0.25f * (float)i;
    params.push_back(t);
  }
  params[3][1] = -0.0f;
  {
    std::FILE *fh = std::fopen(path.c_str(), "wb");
    CHECK(fh != nullptr, "cannot create %s", path.c_str());
    const uint64_t step = 77, n = params.size();
    const float loss = 3.5f;
    std::fwrite("PRICHS02", 1, 8, fh);
    std::fwrite(&step, 8, 1, fh);
    std::fwrite(&loss, 4, 1, fh);
    std::fwrite(&n, 8, 1, fh);
    for (const auto &t : params) {
      const uint64_t len = t.size();
      std::fwrite(&len, 8, 1, fh);
      std::fwrite(t.data(), 4, t.size(), fh);
    }
    std::fclose(fh);
  }
  const prichs_host::Checkpoint ck = prichs_host::load_checkpoint(path);
  CHECK(ck.step == 77 && ck.loss == 3.5f, "header step %llu loss %g", (unsigned long long)ck.step,
        ck.loss);
  CHECK(ck.params.size() == params.size(), "%zu parameters", ck.params.size());
  for (size_t i = 0; i < params.size(); ++i)
    CHECK(ck.params[i].size() == params[i].size() &&
              std::memcmp(ck.params[i].data(), params[i].data(), 4 * params[i].size()) == 0,
          "parameter %zu differs", i);
  // Block 0: router is slot 6, expert 1's down the last slot.
  CHECK(ck.params[prichs_host::block_param_index(0, E, 6)][0] == 106.f, "router slot");
  CHECK(ck.params[prichs_host::block_param_index(0, E, 10 + 3 * 1 + 2)][0] == 115.f, "expert slot");
  expect_error([&] { prichs_host::block_param_index(0, E, 10 + 3 * E); }, "outside a block");
  // A truncated copy (wte's payload cut) fails at open with the reader's message.
  CHECK(::truncate(path.c_str(), 40) == 0, "truncate");
  expect_error([&] { prichs_host::load_checkpoint(path); }, "load_checkpoint");
  std::remove(path.c_str());
}

int main(int argc, char **argv) {
  run("load_checkpoint", test_load_checkpoint);
  if (argc > 1 && std::strcmp(argv[1], "--no-gpu") == 0) {
    // Without a device the constructor's first allocation fails: an Error, not a crash.
    run("engine_creation_without_device_raises", [] {
      expect_error([] { GpuModelEngine e({{4, 3, true}}); }, "hipMalloc");
    });
    // cublas.rs:285-309: no workspace without a device, and matmul_gpu errs.
    run("matmul_gpu_without_device_raises", [] {
      CHECK(prichs_host::get_gpu_workspace() == nullptr, "a workspace without a device");
      std::vector<float> a(8, 1.0f), b(12, 1.0f), c(6, 0.0f);
      expect_error([&] { prichs_host::matmul_gpu(a, b, c, 2, 4, 3); }, "unavailable");
    });
    return g_failed == 0 ? 0 : 1;
  }
  run("persistent_vram_gemm_correctness", test_persistent_vram_gemm_correctness);
  run("matmul_gpu_family", test_matmul_gpu_family);
  run("gpu_rmsnorm_correctness", test_gpu_rmsnorm_correctness);
  run("gpu_batched_attention_execution", test_gpu_batched_attention_execution);
  run("gpu_batched_attention_random", test_gpu_batched_attention_random);
  run("gpu_moe_forward", test_gpu_moe_forward);
  run("error_paths", test_error_paths);
  if (argc > 1) run("moe_config1_parity", [&] { test_moe_config1_parity(argv[1]); });
  std::printf("%s: %d failed\n", g_failed ? "FAILED" : "PASSED", g_failed);
  return g_failed == 0 ? 0 : 1;
}
