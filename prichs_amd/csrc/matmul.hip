// matmul.hip -- general f32 GEMMs on MFMA and the host-slice GEMM workspace.
//
// Replaces the cuBLAS fallback of the reference's prichs-core
// (crates/prichs-cuda/src/cublas.rs): GpuWorkspace (46-166), its matmul_at_b
// (170-219) and matmul_a_bt (221-268), and the process-wide workspace with
// matmul_gpu / matmul_at_b_gpu / matmul_a_bt_gpu (283-327) that
// crates/prichs-core/src/ops.rs:3, 24-31 dispatches every large matmul_2d
// to.  Shapes are arbitrary (no multiple-of-tile requirement): the kernel
// loads its operand tiles with bounds checks and zero fill.
//
// Arithmetic: v_mfma_f32_16x16x4f32 -- full f32 products with f32
// accumulation (the reference's cuBLAS runs TF32 tensor cores,
// engine.rs:370 / cublas.rs:72; this path is at least as precise and stays
// within 1e-4 of the reference's CPU loop, crates/prichs-core/src/ops.rs:
// 33-58, on its shapes).
#include <mutex>
#include <new>

#include "common.hpp"

struct prichs_gpu_workspace {
  std::mutex mu;  // serialises the calls on this handle (the reference's Mutex<GpuWorkspace>)
  int device = 0;
  void *base = nullptr;
  float *a = nullptr, *b = nullptr, *c = nullptr;  // slabs A, B, C
  size_t cap_a = 0, cap_b = 0, cap_c = 0;          // bytes
};

namespace prichs {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kTile = 64;    // output tile (rows and columns)
constexpr int kStepR = 16;   // reduction elements per LDS stage
constexpr int kThreads = 256;

// C[M, N] = sum_r opA(i, r) opB(r, j), row-major C with ldc = N.
//   OP 0 (A B):    opA(i, r) = A[i R + r],  opB(r, j) = B[r N + j]
//   OP 1 (A^T B):  opA(i, r) = A[r M + i],  opB(r, j) = B[r N + j]
//   OP 2 (A B^T):  opA(i, r) = A[i R + r],  opB(r, j) = B[j R + r]
// One workgroup per 64 x 64 tile (tiles numbered row-major over the grid),
// 4 waves of 32 x 32 (2 x 2 MFMA blocks of 16 x 16).  The operand tiles go
// through LDS as [row][r] with a padded row, loaded so that consecutive
// threads read consecutive addresses of whichever index is contiguous.
template <int OP>
__global__ __launch_bounds__(kThreads) void f32_matmul_kernel(const float *__restrict__ A,
                                                              const float *__restrict__ B,
                                                              float *__restrict__ C, long long M,
                                                              long long N, long long R,
                                                              long long n_tiles) {
  __shared__ float As[kTile][kStepR + 1];
  __shared__ float Bs[kTile][kStepR + 1];
  const long long tile = blockIdx.x;
  const long long m0 = (tile / n_tiles) * kTile;
  const long long n0 = (tile % n_tiles) * kTile;
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // Loader coordinates: "rc" = the reduction index is the contiguous one.
  constexpr bool a_rc = OP != 1, b_rc = OP == 2;
  const int a_i = a_rc ? t >> 2 : (t & 15) * 4, a_r = a_rc ? (t & 3) * 4 : t >> 4;
  const int b_j = b_rc ? t >> 2 : (t & 15) * 4, b_r = b_rc ? (t & 3) * 4 : t >> 4;

  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  float ra[4], rb[4];
  auto gload = [&](long long r0) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const long long i = m0 + a_i + (a_rc ? 0 : q), ar = r0 + a_r + (a_rc ? q : 0);
      ra[q] = (i < M && ar < R) ? (OP == 1 ? A[ar * M + i] : A[i * R + ar]) : 0.f;
      const long long j = n0 + b_j + (b_rc ? 0 : q), br = r0 + b_r + (b_rc ? q : 0);
      rb[q] = (j < N && br < R) ? (OP == 2 ? B[j * R + br] : B[br * N + j]) : 0.f;
    }
  };
  auto lstore = [&]() {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      As[a_i + (a_rc ? 0 : q)][a_r + (a_rc ? q : 0)] = ra[q];
      Bs[b_j + (b_rc ? 0 : q)][b_r + (b_rc ? q : 0)] = rb[q];
    }
  };

  // MFMA operands (v_mfma_f32_16x16x4f32): lane l holds A[row l%16][k l/16]
  // and B[k l/16][col l%16]; the result lane holds rows 4 (l/16) + 0..3 of
  // column l%16.
  const int fr = lane & 15, fk = lane >> 4;
  gload(0);
  for (long long r0 = 0; r0 < R; r0 += kStepR) {
    __syncthreads();  // the previous stage's reads are done
    lstore();
    __syncthreads();
    if (r0 + kStepR < R) gload(r0 + kStepR);
#pragma unroll
    for (int ks = 0; ks < kStepR / 4; ++ks) {
      const int kk = ks * 4 + fk;
      float af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = As[wm * 32 + i * 16 + fr][kk];
#pragma unroll
      for (int j = 0; j < 2; ++j) bf[j] = Bs[wn * 32 + j * 16 + fr][kk];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  }

#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const long long col = n0 + wn * 32 + j * 16 + fr;
      if (col >= N) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const long long row = m0 + wm * 32 + i * 16 + 4 * fk + r;
        if (row < M) C[row * N + col] = acc[i][j][r];
      }
    }
}

// Product of two sizes, or SIZE_MAX when it overflows.
size_t mul_sat(size_t a, size_t b) { return (b != 0 && a > SIZE_MAX / b) ? SIZE_MAX : a * b; }

// Output [M, N] and reduction length R of an op in the reference's (m, k, n)
// naming, and the element counts of a, b, c.
struct MatmulDims {
  size_t M, N, R, a_elems, b_elems, c_elems;
};
MatmulDims matmul_dims(int op, size_t m, size_t k, size_t n) {
  MatmulDims d{};
  if (op == PRICHS_MATMUL_ATB) {
    d = {k, n, m, mul_sat(m, k), mul_sat(m, n), mul_sat(k, n)};
  } else if (op == PRICHS_MATMUL_ABT) {
    d = {m, n, k, mul_sat(m, k), mul_sat(n, k), mul_sat(m, n)};
  } else {
    d = {m, n, k, mul_sat(m, k), mul_sat(k, n), mul_sat(m, n)};
  }
  return d;
}

int check_matmul(int op, size_t m, size_t k, size_t n, const char *who, MatmulDims &d) {
  PRICHS_REQUIRE(op == PRICHS_MATMUL_AB || op == PRICHS_MATMUL_ATB || op == PRICHS_MATMUL_ABT,
                 "%s: unknown op %d", who, op);
  d = matmul_dims(op, m, k, n);
  const size_t lim = (size_t)1 << 46;  // element counts: far past any device, no overflow below
  PRICHS_REQUIRE(d.a_elems < lim && d.b_elems < lim && d.c_elems < lim,
                 "%s: m=%zu, k=%zu, n=%zu too large", who, m, k, n);
  return PRICHS_OK;
}

int launch_matmul(int op, const float *a, const float *b, float *c, const MatmulDims &d,
                  hipStream_t s) {
  if (d.M == 0 || d.N == 0) return PRICHS_OK;
  const long long mt = (long long)cdiv(d.M, kTile), nt = (long long)cdiv(d.N, kTile);
  PRICHS_REQUIRE(mt * nt <= (long long)INT32_MAX, "matmul: %zu x %zu output has too many tiles",
                 d.M, d.N);
  const dim3 grid((unsigned)(mt * nt));
  const long long M = (long long)d.M, N = (long long)d.N, R = (long long)d.R;
  if (op == PRICHS_MATMUL_ATB)
    hipLaunchKernelGGL(f32_matmul_kernel<1>, grid, dim3(kThreads), 0, s, a, b, c, M, N, R, nt);
  else if (op == PRICHS_MATMUL_ABT)
    hipLaunchKernelGGL(f32_matmul_kernel<2>, grid, dim3(kThreads), 0, s, a, b, c, M, N, R, nt);
  else
    hipLaunchKernelGGL(f32_matmul_kernel<0>, grid, dim3(kThreads), 0, s, a, b, c, M, N, R, nt);
  PRICHS_LAUNCH_CHECK("matmul launch");
  return PRICHS_OK;
}

// The reference's slab sizes (cublas.rs:77-84): A 16 MB, B 32 MB, C 16 MB.
constexpr size_t kDefaultSlabA = 16u << 20, kDefaultSlabB = 32u << 20, kDefaultSlabC = 16u << 20;

struct Guard {
  int prev = -1;
  bool ok = true;
  explicit Guard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) {
      ok = false;
      return;
    }
    if (prev != dev && hipSetDevice(dev) != hipSuccess) ok = false;
  }
  ~Guard() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

// H2D of a and b into slabs A and B, the product into slab C, D2H, device
// synchronisation: the sequence of GpuWorkspace::matmul (cublas.rs:117-166).
int workspace_run(prichs_gpu_workspace *ws, int op, const float *a, const float *b, float *c,
                  size_t m, size_t k, size_t n, const char *who) {
  PRICHS_REQUIRE(ws != nullptr, "%s: null workspace", who);
  MatmulDims d;
  if (int rc = check_matmul(op, m, k, n, who, d)) return rc;
  PRICHS_REQUIRE((a || d.a_elems == 0) && (b || d.b_elems == 0) && (c || d.c_elems == 0),
                 "%s: null pointer argument", who);
  if (d.a_elems * 4 > ws->cap_a || d.b_elems * 4 > ws->cap_b || d.c_elems * 4 > ws->cap_c)
    return fail(PRICHS_ERR_CAPACITY,
                "%s: matrix dimensions exceed preallocated GPU workspace slabs (m=%zu, k=%zu, "
                "n=%zu; slabs %zu/%zu/%zu bytes)",
                who, m, k, n, ws->cap_a, ws->cap_b, ws->cap_c);
  if (d.c_elems == 0) return PRICHS_OK;
  Guard g(ws->device);
  if (!g.ok) return fail(PRICHS_ERR_HIP, "%s: cannot select device %d", who, ws->device);
  if (d.a_elems)
    PRICHS_HIP_TRY(hipMemcpy(ws->a, a, d.a_elems * 4, hipMemcpyHostToDevice), "workspace: H2D A");
  if (d.b_elems)
    PRICHS_HIP_TRY(hipMemcpy(ws->b, b, d.b_elems * 4, hipMemcpyHostToDevice), "workspace: H2D B");
  if (int rc = launch_matmul(op, ws->a, ws->b, ws->c, d, nullptr)) return rc;
  PRICHS_HIP_TRY(hipMemcpy(c, ws->c, d.c_elems * 4, hipMemcpyDeviceToHost), "workspace: D2H C");
  PRICHS_HIP_TRY(hipDeviceSynchronize(), "workspace: synchronize");
  return PRICHS_OK;
}

// The process-wide workspace of get_gpu_workspace (cublas.rs:283-300):
// created with the reference's slab sizes on first use, on the device that
// is current then; if that fails it stays absent, as the reference's Lazy
// does.  Its calls are serialised by g_ws_mu (the reference's Mutex).
std::mutex g_ws_mu;
prichs_gpu_workspace *g_ws = nullptr;
bool g_ws_tried = false;
char g_ws_error[512] = {0};

prichs_gpu_workspace *global_workspace_locked() {
  if (!g_ws_tried) {
    g_ws_tried = true;
    if (prichs_gpu_workspace_create(0, 0, 0, &g_ws) != PRICHS_OK) {
      g_ws = nullptr;
      snprintf(g_ws_error, sizeof g_ws_error, "%s", prichs_last_error());
    }
  }
  if (!g_ws) set_error("GPU workspace unavailable: %s", g_ws_error);
  return g_ws;
}

// One call on a handle, under that handle's lock: the slabs are shared by
// every caller of the handle (the process-wide one included).
int locked_run(prichs_gpu_workspace *ws, int op, const float *a, const float *b, float *c,
               size_t m, size_t k, size_t n, const char *who) {
  PRICHS_REQUIRE(ws != nullptr, "%s: null workspace", who);
  std::lock_guard<std::mutex> lock(ws->mu);
  return workspace_run(ws, op, a, b, c, m, k, n, who);
}

int global_run(int op, const float *a, const float *b, float *c, size_t m, size_t k, size_t n,
               const char *who) {
  prichs_gpu_workspace *ws;
  {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    ws = global_workspace_locked();
  }
  if (!ws) return PRICHS_ERR_HIP;
  return locked_run(ws, op, a, b, c, m, k, n, who);
}

}  // namespace
}  // namespace prichs

using namespace prichs;

extern "C" int prichs_matmul_f32(int op, const float *a, const float *b, float *c, size_t m,
                                 size_t k, size_t n, void *stream) {
  MatmulDims d;
  if (int rc = check_matmul(op, m, k, n, "matmul_f32", d)) return rc;
  if (d.c_elems == 0) return PRICHS_OK;
  PRICHS_REQUIRE((a || d.a_elems == 0) && (b || d.b_elems == 0) && c,
                 "matmul_f32: null pointer argument");
  return launch_matmul(op, a, b, c, d, as_stream(stream));
}

extern "C" int prichs_gpu_workspace_create(size_t a_bytes, size_t b_bytes, size_t c_bytes,
                                           prichs_gpu_workspace **out) {
  PRICHS_REQUIRE(out != nullptr, "gpu_workspace_create: null output handle");
  *out = nullptr;
  if (a_bytes == 0) a_bytes = kDefaultSlabA;
  if (b_bytes == 0) b_bytes = kDefaultSlabB;
  if (c_bytes == 0) c_bytes = kDefaultSlabC;
  const size_t ra = roundup(a_bytes, 256), rb = roundup(b_bytes, 256), rc_ = roundup(c_bytes, 256);
  PRICHS_REQUIRE(ra >= a_bytes && rb >= b_bytes && rc_ >= c_bytes && ra <= ((size_t)1 << 44) &&
                     rb <= ((size_t)1 << 44) && rc_ <= ((size_t)1 << 44),
                 "gpu_workspace_create: slab sizes too large");
  prichs_gpu_workspace *ws = new (std::nothrow) prichs_gpu_workspace();
  if (!ws) return fail(PRICHS_ERR_CAPACITY, "gpu_workspace_create: out of host memory");
  if (hipGetDevice(&ws->device) != hipSuccess) {
    delete ws;
    return fail(PRICHS_ERR_HIP, "gpu_workspace_create: no HIP device");
  }
  const hipError_t e = hipMalloc(&ws->base, ra + rb + rc_);
  if (e != hipSuccess) {
    delete ws;
    return fail(PRICHS_ERR_CAPACITY, "gpu_workspace_create: hipMalloc(%zu bytes): %s",
                ra + rb + rc_, hipGetErrorString(e));
  }
  char *p = static_cast<char *>(ws->base);
  ws->a = reinterpret_cast<float *>(p);
  ws->b = reinterpret_cast<float *>(p + ra);
  ws->c = reinterpret_cast<float *>(p + ra + rb);
  ws->cap_a = a_bytes;
  ws->cap_b = b_bytes;
  ws->cap_c = c_bytes;
  *out = ws;
  return PRICHS_OK;
}

extern "C" int prichs_gpu_workspace_destroy(prichs_gpu_workspace *ws) {
  if (!ws) return PRICHS_OK;
  {
    // The process-wide workspace lives until the process ends, as the
    // reference's static does (cublas.rs:283-300).
    std::lock_guard<std::mutex> lock(g_ws_mu);
    PRICHS_REQUIRE(ws != g_ws, "gpu_workspace_destroy: the process-wide workspace "
                               "(get_gpu_workspace) is not destroyed by callers");
  }
  int rc = PRICHS_OK;
  {
    Guard g(ws->device);
    if (ws->base && hipFree(ws->base) != hipSuccess)
      rc = fail(PRICHS_ERR_HIP, "gpu_workspace_destroy: hipFree failed");
  }
  delete ws;
  return rc;
}

extern "C" int prichs_gpu_workspace_slabs(const prichs_gpu_workspace *ws, size_t *a_bytes,
                                          size_t *b_bytes, size_t *c_bytes) {
  PRICHS_REQUIRE(ws != nullptr, "gpu_workspace_slabs: null workspace");
  if (a_bytes) *a_bytes = ws->cap_a;
  if (b_bytes) *b_bytes = ws->cap_b;
  if (c_bytes) *c_bytes = ws->cap_c;
  return PRICHS_OK;
}

extern "C" int prichs_gpu_workspace_matmul(prichs_gpu_workspace *ws, const float *a,
                                           const float *b, float *c, size_t m, size_t k,
                                           size_t n) {
  return locked_run(ws, PRICHS_MATMUL_AB, a, b, c, m, k, n, "gpu_workspace_matmul");
}

extern "C" int prichs_gpu_workspace_matmul_at_b(prichs_gpu_workspace *ws, const float *a,
                                                const float *b, float *dw, size_t m, size_t k,
                                                size_t n) {
  return locked_run(ws, PRICHS_MATMUL_ATB, a, b, dw, m, k, n, "gpu_workspace_matmul_at_b");
}

extern "C" int prichs_gpu_workspace_matmul_a_bt(prichs_gpu_workspace *ws, const float *dy,
                                                const float *w, float *dx, size_t m, size_t k,
                                                size_t n) {
  return locked_run(ws, PRICHS_MATMUL_ABT, dy, w, dx, m, k, n, "gpu_workspace_matmul_a_bt");
}

extern "C" prichs_gpu_workspace *prichs_get_gpu_workspace(void) {
  std::lock_guard<std::mutex> lock(g_ws_mu);
  return global_workspace_locked();
}

extern "C" int prichs_matmul_gpu(const float *a, const float *b, float *c, size_t m, size_t k,
                                 size_t n) {
  return global_run(PRICHS_MATMUL_AB, a, b, c, m, k, n, "matmul_gpu");
}

extern "C" int prichs_matmul_at_b_gpu(const float *a, const float *b, float *dw, size_t m,
                                      size_t k, size_t n) {
  return global_run(PRICHS_MATMUL_ATB, a, b, dw, m, k, n, "matmul_at_b_gpu");
}

extern "C" int prichs_matmul_a_bt_gpu(const float *dy, const float *w, float *dx, size_t m,
                                      size_t k, size_t n) {
  return global_run(PRICHS_MATMUL_ABT, dy, w, dx, m, k, n, "matmul_a_bt_gpu");
}
