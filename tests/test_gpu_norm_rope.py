"""GPU parity of RMSNorm, RoPE and the legacy f32 launchers, through the C ABI.

Bars: RoPE is bit-exact (same separately rounded products and sums as
backward.rs:175-184); RMSNorm within 2e-6 relative (parallel sum of squares);
legacy launchers as their reference tests or closed forms state.
"""
import ctypes as C

import numpy as np
import pytest
import torch

from conftest import rel_err
from prichs_amd import _lib as L
from prichs_amd import ops, synth

pytestmark = pytest.mark.gpu


def dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to("cuda").to(dtype)


def host(t):
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


def ptr(t):
    """Raw device address of t.  The caller must keep t referenced until the
    work that uses the address has completed: a temporary freed before the
    launch is enqueued hands its block to the next allocation."""
    return C.c_void_p(t.data_ptr())


@pytest.mark.parametrize("T,d", [(8192, 1536), (7, 100), (33, 1536), (1, 8)])
def test_rmsnorm_against_oracle(cuda, orc, T, d):
    rng = np.random.default_rng(T + d)
    x = (2 * rng.standard_normal((T, d))).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(d)).astype(np.float32)
    ref = orc.rms_norm(x, w, 1e-5)
    out, rstd = ops.rmsnorm(dev(x), dev(w), 1e-5)
    assert rel_err(host(out), ref) <= 2e-6
    x64 = x.astype(np.float64)
    assert rel_err(host(rstd), 1 / np.sqrt((x64 ** 2).mean(1) + 1e-5)) <= 2e-6
    # bf16 in / bf16 out: the input is bf16, the output is the rounded f32 result
    xb = synth.round_bf16(x)
    outb, _ = ops.rmsnorm(dev(xb, torch.bfloat16), dev(w), 1e-5)
    refb = synth.round_bf16(orc.rms_norm(xb, w, 1e-5))
    assert np.abs(host(outb) - refb).max() <= 2 ** -7 * np.abs(refb).max()


def test_legacy_rmsnorm_known_answer(cuda):
    # engine.rs:3041-3053: row [2,2,2,2], w = 1 -> 1.0, rstd 0.5.
    x = dev(np.array([[1, 2, 3, 4], [2, 2, 2, 2]], np.float32))
    w = dev(np.ones(4, np.float32))
    out = torch.empty_like(x)
    rstd = torch.empty(2, device="cuda")
    lib = L.load()
    lib.launch_rmsnorm_forward(ptr(x), ptr(w), ptr(out), ptr(rstd), 2, 4, 1e-5, None)
    assert L.last_error() == "" or "launch" not in L.last_error()
    o = host(out)
    assert np.abs(o[1] - 1.0).max() < 1e-4
    assert abs(host(rstd)[1] - 0.5) < 1e-4


@pytest.mark.parametrize("B,S,H,hd,off", [(4, 2048, 12, 128, 0), (4, 2048, 3, 128, 0),
                                          (1, 37, 2, 6, 5), (2, 16, 1, 10, 0)])
def test_rope_bit_exact(cuda, orc, B, S, H, hd, off):
    rng = np.random.default_rng(S + H + hd)
    cos, sin = orc.precompute_rope_cache(max(S + off, 1024), hd, 500000.0)
    rows = max(S + off, 1024)
    q = rng.standard_normal((B, S, H, hd)).astype(np.float32)
    ref = np.stack([orc.rope_forward(q[b], cos, sin, pos_offset=off) for b in range(B)])
    qd = dev(q)
    ops.rope_(qd, dev(cos), dev(sin), rows, B, S, pos_offset=off)
    np.testing.assert_array_equal(host(qd).view(np.uint32), ref.view(np.uint32))
    qb = synth.round_bf16(q)
    refb = synth.round_bf16(np.stack([orc.rope_forward(qb[b], cos, sin, pos_offset=off)
                                      for b in range(B)]))
    qdb = dev(qb, torch.bfloat16)
    ops.rope_(qdb, dev(cos), dev(sin), rows, B, S, pos_offset=off)
    np.testing.assert_array_equal(host(qdb), refb)
    # sign = -1 undoes the rotation up to rounding
    ops.rope_(qd, dev(cos), dev(sin), rows, B, S, pos_offset=off, sign=-1)
    assert np.abs(host(qd) - q).max() < 1e-5


def test_legacy_rope_identity_and_sign(cuda, orc):
    # engine.rs:2970-2972: cos = 1, sin = 0 leaves Q/K unchanged.
    S, H, hd = 4, 2, 8
    rng = np.random.default_rng(1)
    q = rng.standard_normal((S, H, hd)).astype(np.float32)
    qd = dev(q)
    lib = L.load()
    ones_d, zeros_d = dev(np.ones(S * hd // 2)), dev(np.zeros(S * hd // 2))
    lib.launch_rope(ptr(qd), ptr(ones_d), ptr(zeros_d), S, H, hd, 1, None)
    np.testing.assert_array_equal(host(qd), q)
    cos, sin = orc.precompute_rope_cache(S, hd, 10000.0)
    cos_d, sin_d = dev(cos), dev(sin)
    lib.launch_rope(ptr(qd), ptr(cos_d), ptr(sin_d), S, H, hd, 1, None)
    np.testing.assert_array_equal(host(qd), orc.rope_forward(q, cos, sin))
    # kernels.cu:543 multiplies sin by (float)backward_sign for any int: -1 is
    # the inverse rotation (the oracle's rotation with -sin), 0 scales both
    # elements of each pair by cos, 2 doubles the sine term.
    for sign in (-1, 0, 2):
        qd = dev(q)
        lib.launch_rope(ptr(qd), ptr(cos_d), ptr(sin_d), S, H, hd, sign, None)
        s2 = (np.float32(sign) * sin).astype(np.float32)
        np.testing.assert_array_equal(host(qd), orc.rope_forward(q, cos, s2))


def test_legacy_swiglu_gather_scatter(cuda, orc):
    rng = np.random.default_rng(2)
    n = 10007
    g = (4 * rng.standard_normal(n)).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    out = torch.empty(n, device="cuda")
    lib = L.load()
    gd, ud = dev(g), dev(u)
    lib.launch_swiglu_forward(ptr(gd), ptr(ud), ptr(out), n, None)
    assert rel_err(host(out), orc.swiglu(g, u)) <= 1e-6
    T, d = 50, 24
    src = rng.standard_normal((T, d)).astype(np.float32)
    idx = np.array([3, 7, 7, 0, 49], np.int32)
    idx_d = torch.from_numpy(idx).to("cuda")
    srcd = dev(src)
    gath = torch.empty((len(idx), d), device="cuda")
    lib.launch_moe_gather(ptr(srcd), ptr(idx_d), ptr(gath), len(idx), d, None)
    np.testing.assert_array_equal(host(gath), src[idx])
    uniq = np.array([5, 1, 9], np.int32)
    y = rng.standard_normal((3, d)).astype(np.float32)
    wts = np.array([0.25, 0.5, 2.0], np.float32)
    acc = dev(src)
    y_d, uniq_d, wts_d = dev(y), torch.from_numpy(uniq).to("cuda"), dev(wts)
    assert uniq.min() >= 0 and uniq.max() < T  # indices address rows of acc [T, d]
    lib.launch_moe_scatter_add(ptr(y_d), ptr(uniq_d), ptr(wts_d), ptr(acc), 3, d, None)
    expect = src.copy()
    for i, t in enumerate(uniq):
        expect[t] = expect[t] + wts[i] * y[i]
    np.testing.assert_array_equal(host(acc), expect)


def test_legacy_backward_launchers_run_the_reference_expert_backward(cuda, orc):
    # The reference's per-expert MoE backward (model.rs:1474-1561 driving
    # engine.rs:2242-2789) composed from the four legacy backward launchers,
    # with torch f32 matmuls in place of its cuBLAS SGEMMs and the router VJP
    # (backward.rs:269-287) on the host, reproduces the oracle's gradients
    # (reference weighting) within 1e-4.
    torch.backends.cuda.matmul.allow_tf32 = False
    lib = L.load()
    inp = synth.config_inputs(1)
    T, d, f, E, k = inp.T, inp.d, inp.f, inp.E, inp.k
    rng = np.random.default_rng(6)
    d_out = rng.standard_normal((T, d)).astype(np.float32)
    fwd = orc.moe_forward(inp)
    sel, gw = fwd["sel"], fwd["gw"]
    x = inp.x.astype(np.float32)
    dm = dev(d_out)
    d_normed2 = torch.zeros((T, d), device="cuda")
    grads = {"gate": [np.zeros((d, f), np.float32) for _ in range(E + 1)],
             "up": [np.zeros((d, f), np.float32) for _ in range(E + 1)],
             "down": [np.zeros((f, d), np.float32) for _ in range(E + 1)]}
    scal = np.zeros((T, E), np.float32)

    def expert(j, xe):
        g = xe @ inp.gate[j]
        u = xe @ inp.up[j]
        a = orc.swiglu(g, u)
        return g, u, a, a @ inp.down[j]

    def backward_rows(j, xe, dy, g, u, a):
        wg, wu, wd = dev(inp.gate[j]), dev(inp.up[j]), dev(inp.down[j])
        grads["down"][j] += host(dev(a).T @ dy)
        dact = (dy @ wd.T).contiguous()
        dg, du = torch.empty_like(dact), torch.empty_like(dact)
        gd, ud = dev(g), dev(u)
        lib.launch_swiglu_backward(ptr(dact), ptr(gd), ptr(ud), ptr(dg), ptr(du), dact.numel(), None)
        xd = dev(xe)
        grads["gate"][j] += host(xd.T @ dg)
        grads["up"][j] += host(xd.T @ du)
        return (dg @ wg.T).contiguous(), (du @ wu.T).contiguous()

    for e in range(E):  # gpu_moe_backward_expert, experts ascending
        toks = np.nonzero((sel == e).any(1))[0].astype(np.int32)
        if toks.size == 0:
            continue
        w = np.array([gw[t][list(sel[t]).index(e)] for t in toks], np.float32)
        g, u, a, y = expert(1 + e, x[toks])
        idx_d, w_d, y_d = torch.from_numpy(toks).to("cuda"), dev(w), dev(y)
        n = len(toks)
        dy = torch.empty((n, d), device="cuda")
        lib.launch_moe_backward_gather_weighted(ptr(dm), ptr(idx_d), ptr(w_d), ptr(dy), n, d, None)
        sc = torch.empty(n, device="cuda")
        lib.launch_moe_router_dot(ptr(y_d), ptr(dm), ptr(idx_d), ptr(sc), n, d, None)
        scal[toks, e] = host(sc)
        dxg, dxu = backward_rows(1 + e, x[toks], dy, g, u, a)
        lib.launch_moe_scatter_add_grad(ptr(dxg), ptr(dxu), ptr(idx_d), ptr(w_d), ptr(d_normed2),
                                        n, d, None)
        torch.cuda.synchronize()
    g, u, a, _ = expert(0, x)  # gpu_moe_backward_shared: dY = d_moe
    dxg, dxu = backward_rows(0, x, dm, g, u, a)
    d_normed2 += dxg
    d_normed2 += dxu
    # Router VJP on the host, then gpu_moe_backward_router's two products.
    dlog = np.zeros((T, E), np.float32)
    for t in range(T):
        ws = np.float32(0)
        for j in range(k):
            ws = np.float32(ws + gw[t, j] * scal[t, sel[t, j]])
        for j in range(k):
            dlog[t, sel[t, j]] = gw[t, j] * (scal[t, sel[t, j]] - ws)
    d_router = host(dev(x).T @ dev(dlog))
    d_normed2 += dev(dlog) @ dev(inp.w_router).T
    ref = orc.moe_backward(inp, d_out, dx_weighting=2)
    assert rel_err(host(d_normed2), ref["d_x"]) <= 1e-4
    assert rel_err(d_router, ref["d_router"]) <= 1e-4
    for key in ("gate", "up", "down"):
        for j in range(E + 1):
            assert rel_err(grads[key][j], ref["d_" + key][j]) <= 1e-4, (key, j)


@pytest.mark.parametrize("nbytes", [16, 4096 * 16 + 48, 64 << 20])
def test_hbm_copy_exact(cuda, nbytes):
    # prichs_hbm_copy (the HBM yardstick of the memory-bound stages): every
    # byte copied, nothing past the end touched (whole blocks and a ragged
    # last block).
    print("case: hbm_copy", nbytes, flush=True)
    g = torch.Generator(device="cuda").manual_seed(nbytes % 1000)
    src = torch.randint(-2**31, 2**31 - 1, (nbytes // 4,), dtype=torch.int32, device="cuda",
                        generator=g)
    dst = torch.full((nbytes // 4 + 64,), 0x5A5A5A5A, dtype=torch.int32, device="cuda")
    ops.hbm_copy(src, dst[:nbytes // 4])
    torch.cuda.synchronize()
    assert torch.equal(dst[:nbytes // 4], src)
    assert bool((dst[nbytes // 4:] == 0x5A5A5A5A).all())
