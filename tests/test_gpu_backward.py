"""GPU parity of the MoE backward (prichs_moe_engine_backward) through the C ABI.

Bars (written in each test):
* fp32 engine against the CPU oracle (orc_moe_backward, itself pinned by
  finite differences): max |gpu - ref| / max |ref| <= 1e-4 for d_x and every
  weight gradient, in both dx_weighting modes;
* bf16 engine against the oracle on the same bf16-rounded inputs: <= 2e-2;
* config-2 size (T = 8192, d = 1536, f = 1280): the chain-rule mode against
  torch autograd of an fp32 forward on the GPU's own routing, <= 2e-2;
* determinism, accumulation (beta = 1) and the reference parameter layout:
  bit-exact.
"""
import ctypes as C

import numpy as np
import pytest
import torch

from conftest import rel_err
from prichs_amd import _lib as L
from prichs_amd import moe, synth

pytestmark = pytest.mark.gpu

TOL = {"f32": 1e-4, "bf16": 2e-2}


def dev(a, dtype="f32"):
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to("cuda")
    return t.to(torch.bfloat16) if dtype == "bf16" else t


def host(t):
    torch.cuda.synchronize()
    return t.float().cpu().numpy() if t.dtype == torch.bfloat16 else t.cpu().numpy()


def say(*a):
    print(*a, flush=True)


def make_engine(inp, enable=True):
    eng = moe.MoEEngine(inp.d, inp.f, inp.E, inp.k, 1, inp.dtype, max_tokens=inp.T)
    if enable:
        eng.enable_backward()
    eng.upload(inp.w_router, inp.router_bias, inp.gate, inp.up, inp.down)
    return eng


def zero_grads(inp):
    G = 1 + inp.E
    z = lambda *s: torch.zeros(s, dtype=torch.float32, device="cuda")  # noqa: E731
    return dict(d_router=z(inp.d, inp.E), d_gate=z(G, inp.d, inp.f), d_up=z(G, inp.d, inp.f),
                d_down=z(G, inp.f, inp.d))


def run(eng, inp, d_out, weighting, grads=None):
    x = dev(inp.x, inp.dtype)
    eng.forward(x)
    grads = zero_grads(inp) if grads is None else grads
    d_x = eng.backward(x, dev(d_out, inp.dtype), grads, dx_weighting=weighting,
                       d_x_dtype=torch.float32)
    return d_x, grads


def check_against_oracle(orc, inp, d_out, weighting, got_dx, grads, tol):
    ref = orc.moe_backward(inp, d_out, dx_weighting=weighting)
    errs = {"d_x": rel_err(host(got_dx), ref["d_x"]),
            "d_router": rel_err(host(grads["d_router"]), ref["d_router"])}
    for key in ("d_gate", "d_up", "d_down"):
        g = host(grads[key])
        errs[key] = max(rel_err(g[s], ref[key][s]) for s in range(1 + inp.E))
    say("  errors", {k: f"{v:.2e}" for k, v in errs.items()})
    for k, v in errs.items():
        assert v <= tol, (k, v)


def inputs(T, d, f, E, k, dtype, seed, bias_std=0.3, w_std=0.1):
    inp = synth.make_moe_inputs(T, d, f, E=E, k=k, dtype=dtype, x_norm=True, bias_std=bias_std,
                                w_std=w_std, seed=seed)
    d_out = np.random.default_rng(seed + 11).standard_normal((T, d)).astype(np.float32)
    if dtype == "bf16":
        d_out = synth.round_bf16(d_out)
    return inp, d_out


# ------------------------------------------------------------- fp32 engine --
# Shapes: whole and partial 128-wide weight-gradient tiles (d = 48, 80),
# padded gate/up blocks (f = 80: columns 80..95 of the last block), top-1/3.
@pytest.mark.parametrize("T,d,f,E,k", [(96, 64, 64, 4, 2), (200, 48, 80, 8, 3),
                                       (130, 144, 192, 6, 1)])
@pytest.mark.parametrize("weighting", [1, 2])
def test_backward_f32_matches_oracle(cuda, orc, T, d, f, E, k, weighting):
    say("f32 backward", T, d, f, E, k, "weighting", weighting)
    inp, d_out = inputs(T, d, f, E, k, "f32", seed=T + E)
    eng = make_engine(inp)
    d_x, grads = run(eng, inp, d_out, weighting)
    check_against_oracle(orc, inp, d_out, weighting, d_x, grads, TOL["f32"])


# ------------------------------------------------------------- bf16 engine --
# Config-1 shapes in bf16, a padded f (192: packed columns 384..511 are
# padding), a decode-sized batch whose groups take the skinny GEMM, and a
# batch whose shared group (3000 rows) the weight-gradient kernels split over K.
@pytest.mark.parametrize("T,d,f,E,k", [(512, 256, 128, 8, 2), (300, 128, 192, 8, 2),
                                       (32, 256, 128, 8, 2), (3000, 256, 128, 4, 2)])
@pytest.mark.parametrize("weighting", [1, 2])
def test_backward_bf16_matches_oracle(cuda, orc, T, d, f, E, k, weighting):
    say("bf16 backward", T, d, f, E, k, "weighting", weighting)
    inp, d_out = inputs(T, d, f, E, k, "bf16", seed=T + 3)
    eng = make_engine(inp)
    d_x, grads = run(eng, inp, d_out, weighting)
    check_against_oracle(orc, inp, d_out, weighting, d_x, grads, TOL["bf16"])


@pytest.mark.parametrize("T", [400, 6000])
def test_backward_skewed_routing(cuda, orc, T):
    # Config-3 style bias: experts 0-1 take most rows, some experts may get none.
    # At T = 6000 the hot experts' groups (and the shared one) exceed the
    # weight-gradient kernels' split size, so they are summed from K chunks.
    say("bf16 backward, skewed routing", T)
    inp = synth.make_moe_inputs(T, 128, 128, E=8, k=2, dtype="bf16", bias_std=None,
                                skew_beta=0.5 if T < 1000 else 1.5, w_std=0.1, seed=4)
    d_out = synth.round_bf16(np.random.default_rng(4).standard_normal((T, 128)).astype(np.float32))
    eng = make_engine(inp)
    d_x, grads = run(eng, inp, d_out, 2)
    counts = np.bincount(eng.stash()["selected_experts"].cpu().numpy().ravel(), minlength=8)
    say("  rows per routed expert", counts.tolist())
    if T == 6000:
        assert counts.max() > 2560
    check_against_oracle(orc, inp, d_out, 2, d_x, grads, TOL["bf16"])


# --------------------------------------------------------- host semantics --
@pytest.mark.parametrize("T", [512, 3000])
def test_backward_deterministic_accumulating_and_flat_layout(cuda, T):
    inp, d_out = inputs(T, 256, 128, 8, 2, "bf16", seed=21)
    eng = make_engine(inp)
    say("determinism")
    dx1, g1 = run(eng, inp, d_out, 2)
    dx2, g2 = run(eng, inp, d_out, 2)
    assert torch.equal(dx1, dx2)
    for key in g1:
        assert torch.equal(g1[key], g2[key]), key
    say("accumulation")
    torch.manual_seed(0)
    init = {k: torch.randn_like(v) for k, v in g1.items()}
    _, g3 = run(eng, inp, d_out, 2, grads={k: v.clone() for k, v in init.items()})
    for key in g1:
        assert torch.equal(g3[key], init[key] + g1[key]), key
    say("reference parameter layout")
    G, d, f = 1 + inp.E, inp.d, inp.f
    flat = torch.zeros((G, 3, d * f), dtype=torch.float32, device="cuda")
    d_router = torch.zeros((d, inp.E), dtype=torch.float32, device="cuda")
    x = dev(inp.x, "bf16")
    eng.forward(x)
    dx4 = eng.backward(x, dev(d_out, "bf16"), {"d_router": d_router, "flat": flat},
                       dx_weighting=2, d_x_dtype=torch.float32)
    assert torch.equal(dx4, dx1)
    assert torch.equal(d_router, g1["d_router"])
    assert torch.equal(flat[:, 0].reshape(G, d, f), g1["d_gate"])
    assert torch.equal(flat[:, 1].reshape(G, d, f), g1["d_up"])
    assert torch.equal(flat[:, 2].reshape(G, f, d), g1["d_down"])


@pytest.mark.parametrize("T", [512, 3000])
def test_backward_d_x_in_place_of_x(cuda, T):
    # d_x may be written over x.  The shared expert's rows of x are otherwise
    # read in place after the combine has written d_x, so the engine then
    # copies them as for the routed rows: both routes give the same bits.
    inp, d_out = inputs(T, 256, 128, 8, 2, "bf16", seed=23)
    eng = make_engine(inp)
    say("separate d_x", T)
    x = dev(inp.x, "bf16")
    eng.forward(x)
    g1 = zero_grads(inp)
    dx1 = eng.backward(x, dev(d_out, "bf16"), g1, dx_weighting=2, d_x_dtype=torch.bfloat16)
    say("d_x over x", T)
    x2 = dev(inp.x, "bf16")
    eng.forward(x2)
    g2 = zero_grads(inp)
    eng.backward(x2, dev(d_out, "bf16"), g2, dx_weighting=2, d_x=x2)
    torch.cuda.synchronize()
    assert torch.equal(x2, dx1)
    for key in g1:
        assert torch.equal(g1[key], g2[key]), key


def test_backward_modes_share_weight_gradients(cuda):
    inp, d_out = inputs(256, 128, 128, 8, 2, "bf16", seed=5)
    eng = make_engine(inp)
    dx1, g1 = run(eng, inp, d_out, 1)
    dx2, g2 = run(eng, inp, d_out, 2)
    for key in g1:
        assert torch.equal(g1[key], g2[key]), key
    assert not torch.equal(dx1, dx2)


def test_backward_state_and_argument_errors(cuda):
    inp, d_out = inputs(64, 128, 128, 4, 2, "bf16", seed=9)
    x, go = dev(inp.x, "bf16"), dev(d_out, "bf16")
    grads = zero_grads(inp)
    eng = make_engine(inp, enable=False)
    with pytest.raises(L.PrichsError, match="enable_backward"):
        eng.backward(x, go, grads)
    with pytest.raises(L.PrichsError, match="before upload"):
        eng.enable_backward()
    eng = make_engine(inp)
    with pytest.raises(L.PrichsError, match="forward of this batch"):
        eng.backward(x, go, grads)  # no forward yet
    eng.forward(x)
    with pytest.raises(L.PrichsError, match="forward of this batch"):
        eng.backward(x[:32], go[:32], grads)  # T differs from the forward's
    with pytest.raises(L.PrichsError, match="dx_weighting"):
        eng.backward(x, go, grads, dx_weighting=3)
    eng.backward(x, go, grads)
    with pytest.raises(L.PrichsError, match="forward of this batch"):
        eng.backward(x, go, grads)  # the stash was consumed
    eng.forward(x)
    buf = torch.zeros(inp.T * inp.d + 8, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(L.PrichsError, match="aligned"):
        eng.backward(buf[1:1 + inp.T * inp.d].view(inp.T, inp.d), go, grads)
    eng.forward(x)
    eng.backward(x, go, grads)  # a valid call still works after the errors
    torch.cuda.synchronize()


# ------------------------------------------------------------- full size --
def _autograd_reference(inp, d_out, sel):
    """torch autograd of the layer in fp32 on the GPU, with the selection held
    fixed (the GPU's own, bit-exact with the oracle's routing): the chain-rule
    gradients, derived independently of the backward's formulas."""
    f32 = lambda a: torch.tensor(np.asarray(a, np.float32), device="cuda", requires_grad=True)  # noqa: E731
    x, wr = f32(inp.x), f32(inp.w_router)
    gs, us, ds = ([f32(a) for a in inp.gate], [f32(a) for a in inp.up], [f32(a) for a in inp.down])

    def ffn(xx, j):
        g = xx @ gs[j]
        return (torch.nn.functional.silu(g) * (xx @ us[j])) @ ds[j]

    logits = x @ wr
    gw = torch.softmax(logits.gather(1, sel), dim=1)
    out = ffn(x, 0)
    for e in range(inp.E):
        t, j = torch.nonzero(sel == e, as_tuple=True)
        if t.numel():
            out = out.index_add(0, t, gw[t, j][:, None] * ffn(x[t], 1 + e))
    (out * torch.tensor(d_out, device="cuda")).sum().backward()
    return dict(d_x=x.grad, d_router=wr.grad, d_gate=torch.stack([a.grad for a in gs]),
                d_up=torch.stack([a.grad for a in us]), d_down=torch.stack([a.grad for a in ds]))


def test_backward_config2_against_autograd(cuda):
    inp = synth.config_inputs(2)
    d_out = synth.round_bf16(np.random.default_rng(2).standard_normal((inp.T, inp.d))
                             .astype(np.float32))
    say("config 2 backward", inp.T, inp.d, inp.f)
    eng = make_engine(inp)
    d_x, grads = run(eng, inp, d_out, 1)
    sel = eng.stash()["selected_experts"].long()
    ref = _autograd_reference(inp, d_out, sel)
    errs = {k: rel_err(host(grads[k] if k != "d_x" else d_x), host(ref[k])) for k in ref}
    say("  errors", {k: f"{v:.2e}" for k, v in errs.items()})
    for k, v in errs.items():
        assert v <= TOL["bf16"], (k, v)


@pytest.mark.parametrize("T,dtype", [(512, "bf16"), (32, "bf16"), (200, "f32")])
def test_forward_unchanged_by_enable_backward(cuda, T, dtype):
    # With the backward enabled the gate/up GEMM also stores its
    # pre-activations; the layer output stays bit-identical (tiled, skinny and
    # fp32 kernels).
    say("forward with/without backward", T, dtype)
    inp, _ = inputs(T, 256, 128, 8, 2, dtype, seed=T)
    x = dev(inp.x, dtype)
    outs = []
    for enable in (False, True):
        eng = make_engine(inp, enable=enable)
        outs.append(eng.forward(x))
        torch.cuda.synchronize()
        eng.close()
    assert torch.equal(outs[0], outs[1])


def test_backward_stage_timing(cuda):
    inp, d_out = inputs(512, 256, 128, 8, 2, "bf16", seed=8)
    eng = make_engine(inp)
    eng.set_timing(2)
    for _ in range(2):
        run(eng, inp, d_out, 2)
    ms = eng.backward_stage_ms()
    say("  backward stage ms", ms)
    assert ms["n"] == 2
    assert ms["total"] > 0 and ms["gate_up"] >= 0
    parts = sum(v for kk, v in ms.items() if kk not in ("total", "n"))
    assert abs(parts - ms["total"]) <= 0.05 * ms["total"] + 1e-3
    with pytest.raises(L.PrichsError, match="no timed backward"):
        eng.backward_stage_ms()


@pytest.mark.parametrize("T,dtype", [(512, "bf16"), (3000, "bf16"), (200, "f32")])
def test_backward_beta0_overwrites(cuda, T, dtype):
    # beta = 0 is zero_grads (engine.rs:710-720) followed by the backward: on
    # NaN-filled buffers it must write every element, experts without rows
    # included, and equal beta = 1 on zeroed buffers.  T = 3000 splits the
    # shared group's weight gradients over K.
    say("beta 0", T, dtype)
    inp, d_out = inputs(T, 256, 128, 8, 2, dtype, seed=31)
    inp.router_bias[7] = -1e4  # no token selects expert 7
    eng = make_engine(inp)
    x, go = dev(inp.x, dtype), dev(d_out, dtype)
    eng.forward(x)
    assert int((eng.stash()["selected_experts"] == 7).sum()) == 0
    ref = zero_grads(inp)
    dx1 = eng.backward(x, go, ref, d_x_dtype=torch.float32, beta=1)
    for layout in ("separate", "flat"):
        G, d, f = 1 + inp.E, inp.d, inp.f
        if layout == "separate":
            got = {k: torch.full_like(v, float("nan")) for k, v in ref.items()}
        else:
            got = {"d_router": torch.full_like(ref["d_router"], float("nan")),
                   "flat": torch.full((G, 3, d * f), float("nan"), device="cuda")}
        eng.forward(x)
        dx0 = eng.backward(x, go, got, d_x_dtype=torch.float32, beta=0)
        assert torch.equal(dx0, dx1)
        if layout == "flat":
            fl = got["flat"]
            got = {"d_router": got["d_router"], "d_gate": fl[:, 0].reshape(G, d, f),
                   "d_up": fl[:, 1].reshape(G, d, f), "d_down": fl[:, 2].reshape(G, f, d)}
        for key in ref:
            assert torch.equal(got[key], ref[key]), (layout, key)
        assert not got["d_gate"][8].any() and not got["d_down"][8].any()  # slot 8 = expert 7


def test_backward_empty_batch(cuda):
    inp, _ = inputs(64, 128, 128, 4, 2, "bf16", seed=2)
    eng = make_engine(inp)
    x = dev(inp.x, "bf16")[:0]
    g1 = {k: torch.ones_like(v) for k, v in zero_grads(inp).items()}
    eng.forward(x)
    eng.backward(x, x, g1, beta=1)
    assert all(bool((v == 1).all()) for v in g1.values())
    g0 = {k: torch.full_like(v, float("nan")) for k, v in zero_grads(inp).items()}
    eng.forward(x)
    eng.backward(x, x, g0, beta=0)
    torch.cuda.synchronize()
    assert all(not v.any() for v in g0.values())
