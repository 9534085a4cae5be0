"""Host-slice f32 GEMMs on the GPU: the mirror of the reference's
`prichs_cuda::{GpuWorkspace, get_gpu_workspace, matmul_gpu, matmul_at_b_gpu,
matmul_a_bt_gpu}` (crates/prichs-cuda/src/cublas.rs:46-327; re-exported at
crates/prichs-cuda/src/lib.rs:6-8), which prichs-core's `matmul_2d`,
`matmul_at_b` and `matmul_a_bt` dispatch to (crates/prichs-core/src/ops.rs:3,
24-31, 63-107).

Arguments are numpy float32 arrays in the reference's row-major layouts with
its (m, k, n) naming; every call is synchronous (H2D, the GEMM in
libprichs_hip.so, D2H).  Failures raise PrichsError where the Rust functions
return Err: PRICHS_ERR_CAPACITY when an operand exceeds its slab, and
PRICHS_ERR_HIP ("GPU workspace unavailable") when no GPU workspace exists --
the error on which prichs-core falls back to its CPU loop.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib as L


def _f32(a, size: int, name: str) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    if a.size != size:
        raise ValueError(f"{name} holds {a.size} elements, expected {size}")
    return a


def _ptr(a: np.ndarray):
    return C.c_void_p(a.ctypes.data) if a.size else None


def _out(c, size: int, name: str) -> np.ndarray:
    if not (isinstance(c, np.ndarray) and c.dtype == np.float32 and c.flags.c_contiguous):
        raise TypeError(f"{name} must be a C-contiguous float32 numpy array (written in place)")
    if c.size != size:
        raise ValueError(f"{name} holds {c.size} elements, expected {size}")
    return c


class GpuWorkspace:
    """GpuWorkspace (cublas.rs:46-166): device slabs for A, B and C.

    Sizes are in bytes; 0 selects the reference's 16 MB / 32 MB / 16 MB."""

    def __init__(self, a_bytes: int = 0, b_bytes: int = 0, c_bytes: int = 0, _handle=None):
        lib = L.load()
        self._owned = _handle is None
        if _handle is None:
            h = C.c_void_p()
            L.check(lib.prichs_gpu_workspace_create(a_bytes, b_bytes, c_bytes, C.byref(h)))
            _handle = h
        self._h = _handle

    @property
    def handle(self):
        return self._h

    def slabs(self):
        a, b, c = C.c_size_t(), C.c_size_t(), C.c_size_t()
        L.check(L.load().prichs_gpu_workspace_slabs(self._h, C.byref(a), C.byref(b), C.byref(c)))
        return a.value, b.value, c.value

    def matmul(self, a, b, c, m: int, k: int, n: int) -> None:
        """c [m, n] = a [m, k] @ b [k, n] (cublas.rs:117-166)."""
        a, b, c = _f32(a, m * k, "a"), _f32(b, k * n, "b"), _out(c, m * n, "c")
        L.check(L.load().prichs_gpu_workspace_matmul(self._h, _ptr(a), _ptr(b), _ptr(c), m, k, n))

    def matmul_at_b(self, a, b, dw, m: int, k: int, n: int) -> None:
        """dw [k, n] = a [m, k]^T @ b [m, n], overwritten (cublas.rs:170-219)."""
        a, b, dw = _f32(a, m * k, "a"), _f32(b, m * n, "b"), _out(dw, k * n, "dw")
        L.check(L.load().prichs_gpu_workspace_matmul_at_b(self._h, _ptr(a), _ptr(b), _ptr(dw),
                                                          m, k, n))

    def matmul_a_bt(self, dy, w, dx, m: int, k: int, n: int) -> None:
        """dx [m, n] = dy [m, k] @ w [n, k]^T, overwritten (cublas.rs:221-268)."""
        dy, w, dx = _f32(dy, m * k, "dy"), _f32(w, n * k, "w"), _out(dx, m * n, "dx")
        L.check(L.load().prichs_gpu_workspace_matmul_a_bt(self._h, _ptr(dy), _ptr(w), _ptr(dx),
                                                          m, k, n))

    def close(self) -> None:
        if self._owned and self._h:
            L.check(L.load().prichs_gpu_workspace_destroy(self._h))
        self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def get_gpu_workspace():
    """get_gpu_workspace (cublas.rs:283-300): the process-wide workspace, or
    None when it could not be created."""
    h = L.load().prichs_get_gpu_workspace()
    return GpuWorkspace(_handle=C.c_void_p(h)) if h else None


def matmul_gpu(a, b, c, m: int, k: int, n: int) -> None:
    """matmul_gpu (cublas.rs:302-309) on the process-wide workspace."""
    a, b, c = _f32(a, m * k, "a"), _f32(b, k * n, "b"), _out(c, m * n, "c")
    L.check(L.load().prichs_matmul_gpu(_ptr(a), _ptr(b), _ptr(c), m, k, n))


def matmul_at_b_gpu(a, b, dw, m: int, k: int, n: int) -> None:
    """matmul_at_b_gpu (cublas.rs:311-318)."""
    a, b, dw = _f32(a, m * k, "a"), _f32(b, m * n, "b"), _out(dw, k * n, "dw")
    L.check(L.load().prichs_matmul_at_b_gpu(_ptr(a), _ptr(b), _ptr(dw), m, k, n))


def matmul_a_bt_gpu(dy, w, dx, m: int, k: int, n: int) -> None:
    """matmul_a_bt_gpu (cublas.rs:320-327)."""
    dy, w, dx = _f32(dy, m * k, "dy"), _f32(w, n * k, "w"), _out(dx, m * n, "dx")
    L.check(L.load().prichs_matmul_a_bt_gpu(_ptr(dy), _ptr(w), _ptr(dx), m, k, n))
