"""Pins the oracle's MoE backward (orc_moe_backward) without restating it.

The checks differentiate a float64 forward numerically: central differences of
L = <d_out, moe(x)> with respect to x, the router and every expert matrix,
with routing held where it is (each perturbed point is checked to select the
same experts).  The float64 forward itself is pinned against the oracle's
forward first.  The reference's routed input gradient carries the gate weight
twice (its gather scales dY by w, kernels.cu:926-944, and its scatter scales
again, kernels.cu:971-991); that mode is pinned by differencing a forward in
which each routed expert's output is weighted by w^2 held constant, plus the
router path differenced on its own.
"""
import numpy as np
import pytest

from conftest import rel_err
from prichs_amd import synth

EPS = 1e-5


def _route64(x, w_router, bias, k):
    """Selection on biased logits, softmax weights on raw logits (moe.rs:113-142)."""
    raw = x @ w_router
    adj = raw + bias
    sel = np.argsort(-adj, 1, kind="stable")[:, :k]
    sr = np.take_along_axis(raw, sel, 1)
    e = np.exp(sr - sr.max(1, keepdims=True))
    return sel, e / e.sum(1, keepdims=True), adj


def _ffn64(xx, wg, wu, wd):
    g = xx @ wg
    u = xx @ wu
    return (g / (1 + np.exp(-g)) * u) @ wd


class F64:
    """float64 copy of a MoEInputs whose tensors the differences perturb."""

    def __init__(self, inp):
        self.k, self.E = inp.k, inp.E
        self.x = inp.x.astype(np.float64)
        self.wr = inp.w_router.astype(np.float64)
        self.bias = inp.router_bias.astype(np.float64)
        self.g = [a.astype(np.float64) for a in inp.gate]
        self.u = [a.astype(np.float64) for a in inp.up]
        self.d = [a.astype(np.float64) for a in inp.down]

    def forward(self, x_ffn=None, x_router=None, gw_power=1, gw_fixed=None):
        """Layer output with the expert inputs and the router input separable.

        gw_fixed: use these gate weights (held constant) instead of the router's,
        raised to gw_power."""
        xf = self.x if x_ffn is None else x_ffn
        xr = self.x if x_router is None else x_router
        sel, gw, _ = _route64(xr, self.wr, self.bias, self.k)
        if gw_fixed is not None:
            gw = gw_fixed
        gw = gw ** gw_power
        out = _ffn64(xf, self.g[0], self.u[0], self.d[0])
        for e in range(self.E):
            t, j = np.nonzero(sel == e)
            if t.size:
                out[t] += gw[t, j][:, None] * _ffn64(xf[t], self.g[1 + e], self.u[1 + e],
                                                     self.d[1 + e])
        return out, sel


def _num_grad(loss, arr, sel0, get_sel):
    """Central differences of loss() over every entry of arr (perturbed in place)."""
    gr = np.empty_like(arr)
    flat, gflat = arr.reshape(-1), gr.reshape(-1)
    for i in range(flat.size):
        v = flat[i]
        flat[i] = v + EPS
        lp = loss()
        assert (get_sel() == sel0).all(), "routing moved under the perturbation"
        flat[i] = v - EPS
        lm = loss()
        flat[i] = v
        gflat[i] = (lp - lm) / (2 * EPS)
    return gr


def _setup(T=6, d=8, f=4, E=4, k=2, seed=3, bias_std=0.5):
    inp = synth.make_moe_inputs(T, d, f, E=E, k=k, dtype="f32", x_norm=False,
                                bias_std=bias_std, w_std=0.4, seed=seed)
    rng = np.random.default_rng(seed)
    d_out = rng.standard_normal((T, d)).astype(np.float32)
    m = F64(inp)
    sel0, _, adj = _route64(m.x, m.wr, m.bias, k)
    srt = np.sort(adj, 1)[:, ::-1]
    if k < E:  # margins far above EPS * |weights|, so no selection can flip
        assert (srt[:, k - 1] - srt[:, k]).min() > 1e-3
    return inp, d_out, m, sel0


def test_float64_forward_matches_oracle(orc):
    inp, _, m, sel0 = _setup()
    r = orc.moe_forward(inp)
    out, sel = m.forward()
    np.testing.assert_array_equal(r["sel"], sel0)
    assert rel_err(r["out"], out) < 1e-5


@pytest.mark.parametrize("k,E,bias_std", [(2, 4, 0.5), (1, 3, 0.0), (3, 5, 0.3)])
def test_backward_equals_finite_differences(orc, k, E, bias_std):
    inp, d_out, m, sel0 = _setup(E=E, k=k, bias_std=bias_std, seed=3 + k)
    do64 = d_out.astype(np.float64)
    got = orc.moe_backward(inp, d_out, dx_weighting=1)

    def loss():
        return float((m.forward()[0] * do64).sum())

    def cur_sel():
        return m.forward()[1]

    tol = 1e-5  # measured ~1e-7 (f32 oracle vs float64 differences)
    assert rel_err(got["d_x"], _num_grad(loss, m.x, sel0, cur_sel)) < tol
    assert rel_err(got["d_router"], _num_grad(loss, m.wr, sel0, cur_sel)) < tol
    for j in range(1 + E):
        assert rel_err(got["d_gate"][j], _num_grad(loss, m.g[j], sel0, cur_sel)) < tol, j
        assert rel_err(got["d_up"][j], _num_grad(loss, m.u[j], sel0, cur_sel)) < tol, j
        assert rel_err(got["d_down"][j], _num_grad(loss, m.d[j], sel0, cur_sel)) < tol, j
    # Experts that no token selects get no gradient at all.
    used = set(np.unique(sel0).tolist())
    for e in range(E):
        if e not in used:
            assert not got["d_gate"][1 + e].any() and not got["d_down"][1 + e].any()


def test_reference_weighting_of_routed_input_gradient(orc):
    # dx_weighting = 2: the routed experts' input path sees w^2 (w held
    # constant), the shared expert and the router path are unchanged.
    inp, d_out, m, sel0 = _setup()
    do64 = d_out.astype(np.float64)
    got = orc.moe_backward(inp, d_out, dx_weighting=2)
    _, gw0, _ = _route64(m.x, m.wr, m.bias, inp.k)
    xf = m.x.copy()
    xr = m.x.copy()

    def loss_ffn():
        return float((m.forward(x_ffn=xf, gw_power=2, gw_fixed=gw0)[0] * do64).sum())

    def loss_router():
        return float((m.forward(x_ffn=m.x, x_router=xr)[0] * do64).sum())

    def sel_of(xx):
        return lambda: _route64(xx, m.wr, m.bias, inp.k)[0]

    expect = _num_grad(loss_ffn, xf, sel0, sel_of(xf)) + _num_grad(loss_router, xr, sel0,
                                                                   sel_of(xr))
    assert rel_err(got["d_x"], expect) < 1e-5
    # The true gradient differs from it wherever a routed weight is not 1.
    one = orc.moe_backward(inp, d_out, dx_weighting=1)
    assert rel_err(one["d_x"], expect) > 1e-2
    # Weight gradients do not depend on the mode, bit for bit.
    for key in ("d_router",):
        np.testing.assert_array_equal(got[key], one[key])
    for key in ("d_gate", "d_up", "d_down"):
        for a, b in zip(got[key], one[key]):
            np.testing.assert_array_equal(a, b)


def test_top1_modes_agree(orc):
    # k = 1: the softmax over one selected logit is exactly 1, so both modes and
    # the router gradient coincide (the router gradient is exactly zero).
    inp, d_out, _, _ = _setup(E=3, k=1, bias_std=0.0)
    a = orc.moe_backward(inp, d_out, dx_weighting=1)
    b = orc.moe_backward(inp, d_out, dx_weighting=2)
    np.testing.assert_array_equal(a["d_x"], b["d_x"])
    assert not a["d_router"].any()


def test_gradients_accumulate(orc):
    # Weight gradients add onto what the caller passes (cuBLAS beta = 1 in the
    # reference, engine.rs:2345-2362); d_x is overwritten.
    inp, d_out, _, _ = _setup()
    fresh = orc.moe_backward(inp, d_out)
    rng = np.random.default_rng(9)
    init = dict(d_router=rng.standard_normal(fresh["d_router"].shape).astype(np.float32),
                d_gate=[rng.standard_normal(a.shape).astype(np.float32) for a in fresh["d_gate"]],
                d_up=[rng.standard_normal(a.shape).astype(np.float32) for a in fresh["d_up"]],
                d_down=[rng.standard_normal(a.shape).astype(np.float32) for a in fresh["d_down"]])
    acc = orc.moe_backward(inp, d_out, grads=init)
    np.testing.assert_array_equal(acc["d_x"], fresh["d_x"])
    np.testing.assert_array_equal(acc["d_router"], init["d_router"] + fresh["d_router"])
    for key in ("d_gate", "d_up", "d_down"):
        for a, i, f in zip(acc[key], init[key], fresh[key]):
            np.testing.assert_array_equal(a, i + f)


def test_backward_is_linear_in_d_out(orc):
    # Every gradient is linear in the upstream gradient (routing does not
    # depend on it): scaling d_out by 2 (exact in binary) scales all by 2.
    inp, d_out, _, _ = _setup()
    a = orc.moe_backward(inp, d_out)
    b = orc.moe_backward(inp, 2 * d_out)
    np.testing.assert_array_equal(b["d_x"], 2 * a["d_x"])
    np.testing.assert_array_equal(b["d_router"], 2 * a["d_router"])
    for key in ("d_gate", "d_up", "d_down"):
        for p, q in zip(b[key], a[key]):
            np.testing.assert_array_equal(p, 2 * q)


def test_backward_argument_errors(orc):
    inp, d_out, _, _ = _setup()
    with pytest.raises(RuntimeError):
        orc.moe_backward(inp, d_out, dx_weighting=3)
    two = synth.make_moe_inputs(4, 8, 4, E=4, k=2, n_shared=2, dtype="f32", seed=1)
    with pytest.raises(ValueError):
        orc.moe_backward(two, np.zeros((4, 8), np.float32))
