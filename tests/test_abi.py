"""C-ABI checks that need no GPU: exported symbols, argument validation and
status codes, and the host-side weight packing."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from prichs_amd import _lib as L
from prichs_amd import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "prichs_hip.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b([A-Za-z_][A-Za-z0-9_]*)\s*\(", text)
    skip = {"defined", "sizeof"}
    return sorted({n for n in names if n not in skip and (n.startswith("prichs_") or n.startswith("launch_"))})


@pytest.fixture(scope="module")
def lib():
    return L.load()


def test_library_exports_every_header_function(lib):
    names = header_functions()
    assert len(names) >= 29
    for n in names:
        assert hasattr(lib, n), f"{n} declared in prichs_hip.h but not exported"
    # The ctypes table covers the whole header.
    assert set(names) == set(L.SIGNATURES), set(names) ^ set(L.SIGNATURES)


def test_legacy_signatures_match_reference_extern_block():
    # crates/prichs-cuda/src/engine.rs:89-272 declares these five hot-path launchers.
    text = open(HEADER).read()
    for sig in [
        r"void launch_rmsnorm_forward\(const float \*dev_x, const float \*dev_weight,\s+float \*dev_out, float \*dev_rstd_out, size_t seq_len,\s+size_t hidden_dim, float eps, void \*stream\)",
        r"void launch_swiglu_forward\(const float \*dev_gate, const float \*dev_up,\s+float \*dev_out, size_t total_elements, void \*stream\)",
        r"void launch_rope\(float \*dev_q_or_k, const float \*dev_cos_cache,\s+const float \*dev_sin_cache, size_t seq_len, size_t num_heads,\s+size_t head_dim, int backward_sign, void \*stream\)",
        r"void launch_moe_gather\(const float \*dev_in, const int \*dev_token_indices,\s+float \*dev_out, size_t n_tokens, size_t hidden_dim,\s+void \*stream\)",
        r"void launch_moe_scatter_add\(const float \*dev_exp_out,\s+const int \*dev_token_indices,\s+const float \*dev_weights, float \*dev_accum_out,\s+size_t n_tokens, size_t hidden_dim, void \*stream\)",
    ]:
        assert re.search(sig, text), sig


def test_legacy_backward_signatures_match_reference_extern_block():
    # engine.rs:152-160 and 244-271 declare the backward launchers.
    text = open(HEADER).read()
    for sig in [
        r"void launch_swiglu_backward\(const float \*dev_dact, const float \*dev_gate,\s+const float \*dev_up, float \*dev_dgate, float \*dev_dup,\s+size_t total_elements, void \*stream\)",
        r"void launch_moe_backward_gather_weighted\(const float \*dev_d_moe,\s+const int \*dev_token_indices,\s+const float \*dev_weights, float \*dev_d_y_e,\s+size_t n_tokens, size_t hidden_dim,\s+void \*stream\)",
        r"void launch_moe_router_dot\(const float \*dev_exp_out, const float \*dev_d_moe,\s+const int \*dev_token_indices, float \*dev_scalars_out,\s+size_t n_tokens, size_t hidden_dim, void \*stream\)",
        r"void launch_moe_scatter_add_grad\(const float \*dev_d_x_e, const float \*dev_d_x_e_tmp,\s+const int \*dev_token_indices,\s+const float \*dev_weights, float \*dev_d_normed2,\s+size_t n_tokens, size_t hidden_dim, void \*stream\)",
    ]:
        assert re.search(sig, text), sig


def test_legacy_backward_launchers_record_null_arguments(lib):
    p = C.c_void_p(16)
    for call, name in [
        (lambda: lib.launch_swiglu_backward(None, p, p, p, p, 8, None), "launch_swiglu_backward"),
        (lambda: lib.launch_moe_backward_gather_weighted(p, None, p, p, 2, 4, None),
         "launch_moe_backward_gather_weighted"),
        (lambda: lib.launch_moe_router_dot(p, p, p, None, 2, 4, None), "launch_moe_router_dot"),
        (lambda: lib.launch_moe_scatter_add_grad(p, p, p, p, None, 2, 4, None),
         "launch_moe_scatter_add_grad"),
    ]:
        lib.prichs_clear_error()
        call()
        assert name in L.last_error() and "null" in L.last_error()
    lib.prichs_clear_error()
    lib.launch_moe_router_dot(None, None, None, None, 0, 4, None)  # empty: no-op, no error
    assert L.last_error() == ""


def test_abi_version_and_error_slot(lib):
    assert lib.prichs_abi_version() == 200
    lib.prichs_clear_error()
    assert L.last_error() == ""


def _expect(status, code, needle=None):
    assert status == code, (status, L.last_error())
    if needle:
        assert needle in L.last_error()


def test_hbm_copy_argument_errors(lib):
    # Validation runs before any device query: these fail the same way with
    # or without a GPU.
    p, q = C.c_void_p(4096), C.c_void_p(1 << 20)
    _expect(lib.prichs_hbm_copy(p, q, 24, None), L.PRICHS_ERR_INVALID_ARGUMENT, "multiple of 16")
    _expect(lib.prichs_hbm_copy(None, q, 32, None), L.PRICHS_ERR_INVALID_ARGUMENT, "null")
    _expect(lib.prichs_hbm_copy(C.c_void_p(4104), q, 32, None), L.PRICHS_ERR_INVALID_ARGUMENT,
            "aligned")
    _expect(lib.prichs_hbm_copy(p, C.c_void_p(4096 + 16), 64, None),
            L.PRICHS_ERR_INVALID_ARGUMENT, "overlap")
    assert lib.prichs_hbm_copy(None, None, 0, None) == L.PRICHS_OK  # empty: no-op


def test_router_argument_errors(lib):
    p = C.c_void_p(16)  # never dereferenced: validation fails first
    args = lambda E, k, T=4, d=8, x=p, dt=L.DTYPE_F32: (x, dt, p, p, None, 0, T, d, E, k, p, p, p, p, None)
    _expect(lib.prichs_router_topk(*args(0, 1)), L.PRICHS_ERR_INVALID_ARGUMENT, "E=0")
    _expect(lib.prichs_router_topk(*args(65, 2)), L.PRICHS_ERR_INVALID_ARGUMENT, "E=65")
    _expect(lib.prichs_router_topk(*args(8, 9)), L.PRICHS_ERR_INVALID_ARGUMENT, "k=9")
    _expect(lib.prichs_router_topk(*args(8, 0)), L.PRICHS_ERR_INVALID_ARGUMENT, "k=0")
    _expect(lib.prichs_router_topk(*args(8, 2, dt=7)), L.PRICHS_ERR_INVALID_ARGUMENT, "dtype")
    _expect(lib.prichs_router_topk(*args(8, 2, x=None)), L.PRICHS_ERR_INVALID_ARGUMENT, "null")
    # T * k overflow of the int32 row space
    _expect(lib.prichs_router_topk(*args(8, 2, T=2**31)), L.PRICHS_ERR_INVALID_ARGUMENT, "too large")
    # T == 0 is a valid empty batch
    assert lib.prichs_router_topk(*args(8, 2, T=0)) == L.PRICHS_OK
    assert lib.prichs_router_num_blocks(8192, 8) == 256
    assert lib.prichs_router_num_blocks(8192, 65) == 0


def test_permute_and_combine_argument_errors(lib):
    p = C.c_void_p(16)
    _expect(lib.prichs_permute(p, p, p, 10, 8, 0, p, p, p, p, None), L.PRICHS_ERR_INVALID_ARGUMENT, "k=0")
    _expect(lib.prichs_permute(p, p, p, 10, 8, 2, None, p, p, p, None), L.PRICHS_ERR_INVALID_ARGUMENT, "offsets")
    _expect(lib.prichs_moe_combine(p, 0, p, p, p, 10, 16, 9, 1, p, 0, None), L.PRICHS_ERR_INVALID_ARGUMENT, "k=9")
    _expect(lib.prichs_moe_combine(None, 0, p, p, p, 10, 16, 2, 1, p, 0, None), L.PRICHS_ERR_INVALID_ARGUMENT, "null")
    assert lib.prichs_moe_combine(None, 0, None, None, None, 0, 16, 2, 1, None, 0, None) == L.PRICHS_OK


def test_gemm_shape_errors(lib):
    p = C.c_void_p(16)
    _expect(lib.prichs_grouped_gate_up_swiglu(p, p, p, 9, 100, p, 1000, 1280, L.DTYPE_BF16, p, None),
            L.PRICHS_ERR_UNSUPPORTED, "multiples of 64")
    _expect(lib.prichs_grouped_down(p, p, 66, 100, p, 1536, 1280, L.DTYPE_BF16, p, None),
            L.PRICHS_ERR_INVALID_ARGUMENT, "G=66")
    _expect(lib.prichs_grouped_down(p, p, 9, 100, p, 1536, 1280, L.DTYPE_F32, None, None),
            L.PRICHS_ERR_INVALID_ARGUMENT, "null")


def test_norm_rope_argument_errors(lib):
    p = C.c_void_p(16)
    _expect(lib.prichs_rope_forward(p, 0, p, p, 10, 1, 11, 2, 8, 0, 1, None), L.PRICHS_ERR_INVALID_ARGUMENT, "cache")
    _expect(lib.prichs_rope_forward(p, 0, p, p, 10, 1, 4, 2, 7, 0, 1, None), L.PRICHS_ERR_INVALID_ARGUMENT, "even")
    _expect(lib.prichs_rope_forward(p, 0, p, p, 10, 1, 4, 2, 8, 0, 2, None), L.PRICHS_ERR_INVALID_ARGUMENT, "sign")
    _expect(lib.prichs_rmsnorm_forward(p, 3, p, p, 0, None, 4, 8, 1e-5, None), L.PRICHS_ERR_INVALID_ARGUMENT, "dtype")


def test_engine_argument_errors(lib):
    h = C.c_void_p()
    _expect(lib.prichs_moe_engine_create(1536, 1280, 8, 2, 2, L.DTYPE_BF16, 16, C.byref(h)),
            L.PRICHS_ERR_INVALID_ARGUMENT, "n_shared")
    _expect(lib.prichs_moe_engine_create(1536, 1280, 8, 3, 1, L.DTYPE_BF16, 0, C.byref(h)),
            L.PRICHS_ERR_INVALID_ARGUMENT, "max_tokens")
    _expect(lib.prichs_moe_engine_create(100, 1280, 8, 2, 1, L.DTYPE_BF16, 16, C.byref(h)),
            L.PRICHS_ERR_UNSUPPORTED, "multiples of 64")
    _expect(lib.prichs_moe_engine_create(1536, 1280, 8, 9, 1, L.DTYPE_BF16, 16, C.byref(h)),
            L.PRICHS_ERR_INVALID_ARGUMENT, "k=9")
    _expect(lib.prichs_moe_engine_create(1536, 1280, 8, 2, 1, L.DTYPE_BF16, 2**31, C.byref(h)),
            L.PRICHS_ERR_INVALID_ARGUMENT, "max_tokens")
    _expect(lib.prichs_moe_engine_forward(None, None, 4, None, 0, None, 0, None),
            L.PRICHS_ERR_INVALID_ARGUMENT, "null engine")
    assert lib.prichs_moe_engine_destroy(None) == L.PRICHS_OK
    _expect(lib.prichs_moe_engine_enable_backward(None), L.PRICHS_ERR_INVALID_ARGUMENT,
            "null engine")
    g = L.MoEGrads()
    _expect(lib.prichs_moe_engine_backward(None, None, None, 4, None, L.DTYPE_F32, C.byref(g), 2,
                                           None), L.PRICHS_ERR_INVALID_ARGUMENT, "null pointer")


def test_matmul_argument_errors(lib):
    p = C.c_void_p(16)
    _expect(lib.prichs_matmul_f32(3, p, p, p, 2, 2, 2, None), L.PRICHS_ERR_INVALID_ARGUMENT,
            "unknown op")
    _expect(lib.prichs_matmul_f32(L.MATMUL_AB, None, p, p, 2, 2, 2, None),
            L.PRICHS_ERR_INVALID_ARGUMENT, "null")
    _expect(lib.prichs_matmul_f32(L.MATMUL_ABT, p, p, p, 2**40, 2**20, 2, None),
            L.PRICHS_ERR_INVALID_ARGUMENT, "too large")
    # an empty output is a no-op before any pointer is used
    assert lib.prichs_matmul_f32(L.MATMUL_AB, None, None, None, 0, 5, 7, None) == L.PRICHS_OK
    assert lib.prichs_matmul_f32(L.MATMUL_ATB, None, None, None, 5, 0, 7, None) == L.PRICHS_OK
    for fn in (lib.prichs_gpu_workspace_matmul, lib.prichs_gpu_workspace_matmul_at_b,
               lib.prichs_gpu_workspace_matmul_a_bt):
        _expect(fn(None, p, p, p, 2, 2, 2), L.PRICHS_ERR_INVALID_ARGUMENT, "null workspace")
    _expect(lib.prichs_gpu_workspace_slabs(None, None, None, None), L.PRICHS_ERR_INVALID_ARGUMENT,
            "null workspace")
    _expect(lib.prichs_gpu_workspace_create(0, 0, 0, None), L.PRICHS_ERR_INVALID_ARGUMENT, "null")
    assert lib.prichs_gpu_workspace_destroy(None) == L.PRICHS_OK


def test_process_wide_workspace_absent_without_a_gpu(lib):
    # get_gpu_workspace is None when the workspace cannot be created
    # (cublas.rs:285-296), and matmul_gpu then fails with "GPU workspace
    # unavailable" (cublas.rs:302-309) -- prichs-core's cue to use its CPU loop.
    import torch

    if torch.cuda.device_count() > 0:
        pytest.skip("a GPU is visible: the workspace exists")
    from prichs_amd import workspace

    assert lib.prichs_get_gpu_workspace() is None
    assert "unavailable" in L.last_error()
    assert workspace.get_gpu_workspace() is None
    out = np.zeros(6, np.float32)
    with pytest.raises(L.PrichsError) as e:
        workspace.matmul_gpu(np.ones(8, np.float32), np.ones(12, np.float32), out, 2, 4, 3)
    assert e.value.status == L.PRICHS_ERR_HIP and "unavailable" in e.value.message
    assert not out.any()


# ----------------------------------------------------------------- packing --
@pytest.mark.parametrize("dtype", [L.DTYPE_F32, L.DTYPE_BF16])
def test_pack_gate_up_layout(lib, dtype):
    from prichs_amd import ops

    rng = np.random.default_rng(7)
    d, f = 128, 192  # f not a multiple of the padded block: exercises zero padding
    gate = rng.standard_normal((d, f)).astype(np.float32)
    up = rng.standard_normal((d, f)).astype(np.float32)
    il = lib.prichs_gate_up_interleave(dtype)
    packed = ops.pack_gate_up(gate, up, dtype)
    np_ = packed.shape[0]
    # whole [il gate | il up] blocks, zero-padded to the kernel's N tile
    assert np_ % (2 * il) == 0 and np_ >= 2 * (-(-f // il) * il)
    assert np_ % (256 if dtype == L.DTYPE_BF16 else 128) == 0
    vals = ops.packed_rows(packed, dtype)
    vals = synth.from_bf16_bits(vals) if dtype == L.DTYPE_BF16 else vals
    rnd = synth.round_bf16 if dtype == L.DTYPE_BF16 else (lambda a: a)
    for p in range(np_):
        b, q = divmod(p, 2 * il)
        src, col = (gate, il * b + q) if q < il else (up, il * b + q - il)
        expect = rnd(src[:, col]) if col < f else np.zeros(d, np.float32)
        np.testing.assert_array_equal(vals[p], expect)


@pytest.mark.parametrize("dtype", [L.DTYPE_F32, L.DTYPE_BF16])
def test_pack_down_layout(lib, dtype):
    from prichs_amd import ops

    rng = np.random.default_rng(8)
    d, f = 320, 64
    down = rng.standard_normal((f, d)).astype(np.float32)
    packed = ops.pack_down(down, dtype)
    assert packed.shape == (512, f)
    vals = ops.packed_rows(packed, dtype)
    vals = synth.from_bf16_bits(vals) if dtype == L.DTYPE_BF16 else vals
    rnd = synth.round_bf16 if dtype == L.DTYPE_BF16 else (lambda a: a)
    np.testing.assert_array_equal(vals[:d], rnd(down.T.copy()))
    assert not vals[d:].any()


def test_bf16_rounding_matches_numpy_model(lib):
    # The library's host bf16 conversion (used by packing) rounds to nearest even.
    from prichs_amd import ops

    vals = np.array([1.0, 1.00390625, 1.005859375, 1.0 + 2**-8 + 2**-9, -3.14159, 65504.0,
                     1e-30, 3.0e38, np.inf, -np.inf], np.float32)
    d = 64
    gate = np.zeros((d, 64), np.float32)
    gate[: len(vals), 0] = vals
    packed = ops.packed_rows(ops.pack_gate_up(gate, gate, L.DTYPE_BF16), L.DTYPE_BF16)
    np.testing.assert_array_equal(synth.from_bf16_bits(packed[0]), synth.round_bf16(gate[:, 0]))
