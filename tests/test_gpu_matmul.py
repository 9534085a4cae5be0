"""GPU parity of the general f32 GEMMs (prichs_matmul_f32) and the host-slice
workspace API that replaces prichs-cuda's GpuWorkspace / matmul_gpu /
matmul_at_b_gpu / matmul_a_bt_gpu (crates/prichs-cuda/src/cublas.rs:46-327),
through the C ABI.

Bar: max |gpu - ref| / max |ref| <= 1e-4 against the CPU oracle (the
reference's CPU loops, crates/prichs-core/src/ops.rs:33-107), and the
reference's own GEMM known-answer test (engine.rs:2877-2936) within its 1e-4
absolute tolerance.
"""
import numpy as np
import pytest
import torch

from conftest import rel_err
from prichs_amd import _lib as L
from prichs_amd import ops, workspace

pytestmark = pytest.mark.gpu

TOL = 1e-4


def say(*a):
    print(*a, flush=True)


def kat():
    w = np.arange(1, 13, dtype=np.float32).reshape(4, 3)
    x = np.array([[1.0, 0.5, 0.2, 0.1], [2.0, 1.0, 0.0, -1.0]], np.float32)
    dy = np.array([[0.5, -0.5, 1.0], [1.0, 2.0, -1.0]], np.float32)
    return x, w, dy


def cpu_ref(op, a, b, orc):
    if op == L.MATMUL_AB:
        return orc.matmul_2d(a, b)
    if op == L.MATMUL_ATB:
        return orc.matmul_at_b(a, b)
    return orc.matmul_a_bt(a, b)


def test_reference_gemm_known_answer_through_matmul_gpu(cuda, orc):
    # engine.rs:2881-2936: forward x W, backward-data dY W^T, backward-weight
    # x^T dY on the KAT's data; every element within 1e-4 of the CPU loops.
    say("case: KAT through prichs_matmul_gpu / _a_bt_gpu / _at_b_gpu")
    x, w, dy = kat()
    out = np.zeros((2, 3), np.float32)
    workspace.matmul_gpu(x, w, out, 2, 4, 3)
    assert np.abs(out - orc.matmul_2d(x, w)).max() < 1e-4
    dx = np.zeros((2, 4), np.float32)
    workspace.matmul_a_bt_gpu(dy, w, dx, 2, 3, 4)
    assert np.abs(dx - orc.matmul_a_bt(dy, w)).max() < 1e-4
    dw = np.full((4, 3), 7.0, np.float32)  # the GPU path overwrites (beta = 0)
    workspace.matmul_at_b_gpu(x, dy, dw, 2, 4, 3)
    assert np.abs(dw - orc.matmul_at_b(x, dy)).max() < 1e-4


def test_process_wide_workspace_has_the_reference_slabs(cuda):
    # cublas.rs:77-84: slab A 16 MB, B 32 MB, C 16 MB; one instance per process.
    ws = workspace.get_gpu_workspace()
    assert ws is not None
    assert ws.slabs() == (16 << 20, 32 << 20, 16 << 20)
    assert workspace.get_gpu_workspace().handle.value == ws.handle.value


def test_process_wide_workspace_is_locked_and_not_destroyed(cuda, orc):
    # The reference hands its workspace out only as &Mutex<GpuWorkspace>
    # (cublas.rs:283-300): every use is locked and the static lives on.  Here
    # destroying the process-wide handle is refused, and threads that share
    # its slabs -- through the handle and through matmul_gpu -- each get their
    # own product (a race on slabs A/B/C would mix the operands of two calls).
    import threading

    say("case: process-wide workspace: destroy refused, 4 threads sharing the slabs")
    ws = workspace.get_gpu_workspace()
    assert L.load().prichs_gpu_workspace_destroy(ws.handle) == L.PRICHS_ERR_INVALID_ARGUMENT
    assert "process-wide" in L.last_error()
    rng = np.random.default_rng(11)
    jobs = []
    for t in range(4):
        m, k, n = 48 + 16 * t, 64 + 8 * t, 40 + 24 * t
        a = rng.standard_normal((m, k)).astype(np.float32)
        b = rng.standard_normal((k, n)).astype(np.float32)
        jobs.append((m, k, n, a, b, orc.matmul_2d(a, b)))
    errors = []

    def run(t):
        m, k, n, a, b, ref = jobs[t]
        for i in range(25):
            out = np.zeros((m, n), np.float32)
            if (i + t) % 2:
                ws.matmul(a, b, out, m, k, n)
            else:
                workspace.matmul_gpu(a, b, out, m, k, n)
            e = rel_err(out, ref)
            if not e <= TOL:
                errors.append((t, i, e))
                return

    threads = [threading.Thread(target=run, args=(t,)) for t in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors, errors
    # the handle still works after the refused destroy
    m, k, n, a, b, ref = jobs[0]
    out = np.zeros((m, n), np.float32)
    ws.matmul(a, b, out, m, k, n)
    assert rel_err(out, ref) <= TOL


def test_capacity_error_before_any_copy(cuda):
    # The router shape's A operand (8192 x 1536 f32 = 48 MB) exceeds slab A:
    # PRICHS_ERR_CAPACITY, the reference's "exceed preallocated GPU workspace
    # slabs" bail (cublas.rs:126-128), on which prichs-core falls back to the CPU.
    say("case: capacity error")
    a = np.zeros(8192 * 1536, np.float32)
    b = np.zeros(1536 * 8, np.float32)
    c = np.full(8192 * 8, 3.0, np.float32)
    with pytest.raises(L.PrichsError) as e:
        workspace.matmul_gpu(a, b, c, 8192, 1536, 8)
    assert e.value.status == L.PRICHS_ERR_CAPACITY
    assert (c == 3.0).all()  # nothing written


@pytest.mark.parametrize("shape", [(8192, 1536, 8), (2048, 1536, 1280)],
                         ids=["router_8192x1536x8", "expert_2048x1536x1280"])
def test_matmul_against_oracle_at_config2_shapes(cuda, orc, shape):
    # matmul_2d of the router ([T, d] x [d, E]) and of one expert's gate
    # projection ([M_e, d] x [d, f]) at configuration 2, through a workspace
    # sized for them, against the oracle's f32 loop (ops.rs:44-58).
    m, k, n = shape
    say(f"case: workspace matmul {shape}")
    rng = np.random.default_rng(11)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = (rng.standard_normal((k, n)) * 0.02).astype(np.float32)
    with workspace.GpuWorkspace(m * k * 4, k * n * 4, m * n * 4) as ws:
        c = np.empty((m, n), np.float32)
        ws.matmul(a, b, c, m, k, n)
    err = rel_err(c, orc.matmul_2d(a, b))
    say(f"  rel err {err:.2e}")
    assert err <= TOL


@pytest.mark.parametrize("op", [L.MATMUL_AB, L.MATMUL_ATB, L.MATMUL_ABT],
                         ids=["ab", "at_b", "a_bt"])
def test_ragged_shapes_all_ops(cuda, orc, op):
    # Sizes that are not multiples of the kernel's 64 x 64 x 16 tile, with an
    # empty reduction (k = 0: c = 0, as the reference's loops leave it) and
    # single rows / columns; through the device entry point and the workspace.
    rng = np.random.default_rng(3 + op)
    shapes = [(1, 1, 1), (3, 5, 7), (17, 1, 65), (65, 63, 17), (100, 129, 1), (1, 300, 130),
              (257, 70, 33), (5, 0, 9)]
    with workspace.GpuWorkspace(1 << 22, 1 << 22, 1 << 22) as ws:
        for (m, k, n) in shapes:
            say(f"case: op {op} m={m} k={k} n={n}")
            a = rng.standard_normal((m, k)).astype(np.float32)
            if op == L.MATMUL_AB:
                b, cshape = rng.standard_normal((k, n)).astype(np.float32), (m, n)
            elif op == L.MATMUL_ATB:
                b, cshape = rng.standard_normal((m, n)).astype(np.float32), (k, n)
            else:
                b, cshape = rng.standard_normal((n, k)).astype(np.float32), (m, n)
            ref = cpu_ref(op, a, b, orc)
            # device pointers
            out = torch.full(cshape, float("nan"), device="cuda")
            ops.matmul_f32(op, torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda(), out=out)
            got = out.cpu().numpy()
            if ref.size:
                assert rel_err(got, ref) <= TOL if np.abs(ref).max() > 0 else not got.any()
            # host slices
            c = np.full(cshape, np.nan, np.float32)
            fn = {L.MATMUL_AB: ws.matmul, L.MATMUL_ATB: ws.matmul_at_b,
                  L.MATMUL_ABT: ws.matmul_a_bt}[op]
            fn(a, b, c, m, k, n)
            np.testing.assert_array_equal(c, got)  # same kernel, same bits


def test_matmul_device_entry_on_stream_and_big_reduction(cuda, orc):
    # A long reduction (k = 4097) on a non-default stream: the result is the
    # oracle's within 1e-4 and every element is written.
    rng = np.random.default_rng(5)
    m, k, n = 70, 4097, 90
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        ta, tb = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
        out = ops.matmul_f32(L.MATMUL_AB, ta, tb, stream=s)
    s.synchronize()
    assert rel_err(out.cpu().numpy(), orc.matmul_2d(a, b)) <= TOL
