"""prichs_moe_forward_noalloc (the MoE forward that allocates nothing, its
intermediates in the library's static device scratch) against
prichs_moe_engine_forward, through the C ABI.

Bar: bit-exact -- the two entry points run the same kernels in the same
order, so routing, the permutation and every output bit agree.  Each case
makes two calls in a row, the second with fewer tokens, so the second runs
on the scratch contents the first left behind.
"""
import ctypes as C

import numpy as np
import pytest
import torch

from prichs_amd import _lib as L
from prichs_amd import moe, ops, synth

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def dev(a, dtype="f32"):
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to("cuda")
    return t.to(torch.bfloat16) if dtype == "bf16" else t


def packed_weights(inp):
    # group order of the grouped GEMMs: routed 0..E-1, then the shared expert
    order = list(range(inp.n_shared, inp.n_shared + inp.E)) + list(range(inp.n_shared))
    gu = ops.to_device_packed([ops.pack_gate_up(inp.gate[j], inp.up[j], inp.dtype) for j in order],
                              inp.dtype)
    dn = ops.to_device_packed([ops.pack_down(inp.down[j], inp.dtype) for j in order], inp.dtype)
    return gu, dn


def noalloc_forward(inp, x, wr, rb, gu, dn, out, concept=None):
    lib = L.load()
    nc = 0 if concept is None else concept.numel()
    return lib.prichs_moe_forward_noalloc(
        ops._p(x), x.shape[0], inp.d, inp.f, inp.E, inp.k, inp.n_shared, ops.dtype_code(inp.dtype),
        ops._p(wr), ops._p(rb), ops._p(gu), ops._p(dn), ops._p(concept), nc, ops._p(out),
        ops.dtype_code(out), ops._stream())


@pytest.mark.parametrize("cfg,T1,T2", [(2, 1200, 37), (4, 32, 5), (1, 512, 100)],
                         ids=["config2_dims_1200_then_37", "decode_32_then_5", "f32_config1_512_then_100"])
def test_noalloc_forward_matches_engine(cuda, cfg, T1, T2):
    inp = synth.config_inputs(cfg, T=T1)
    say(f"case: noalloc cfg {cfg} T {T1} then {T2} ({inp.dtype})")
    eng = moe.MoEEngine(inp.d, inp.f, inp.E, inp.k, inp.n_shared, inp.dtype, max_tokens=T1)
    eng.upload(inp.w_router, inp.router_bias, inp.gate, inp.up, inp.down)
    gu, dn = packed_weights(inp)
    wr, rb = dev(inp.w_router), dev(inp.router_bias)
    x = dev(inp.x, inp.dtype)
    for T in (T1, T2):
        xs = x[:T].contiguous()
        ref = eng.forward(xs)
        ref_sel = eng.stash(["selected_experts"])["selected_experts"]
        out = torch.full_like(ref, float("nan"))
        rc = noalloc_forward(inp, xs, wr, rb, gu, dn, out)
        assert rc == L.PRICHS_OK, L.last_error()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16) if out.dtype == torch.bfloat16 else out.view(torch.int32),
                           ref.view(torch.int16) if ref.dtype == torch.bfloat16 else ref.view(torch.int32)), T
        say(f"  T={T}: bit-exact ({ref_sel.shape[0]} tokens routed)")
    eng.close()


def test_noalloc_rejects_a_batch_past_the_scratch(cuda):
    # At config-2 dims 4096 tokens need ~70 MB of intermediates: refused with
    # PRICHS_ERR_CAPACITY before any GPU work, and out is untouched.
    inp = synth.config_inputs(4, T=4096)
    say("case: noalloc capacity")
    gu, dn = packed_weights(inp)
    wr, rb = dev(inp.w_router), dev(inp.router_bias)
    x = dev(inp.x, inp.dtype)
    out = torch.zeros_like(x)
    rc = noalloc_forward(inp, x, wr, rb, gu, dn, out)
    assert rc == L.PRICHS_ERR_CAPACITY and "scratch" in L.last_error()
    torch.cuda.synchronize()
    assert not out.any()


@pytest.mark.parametrize("cfg,T", [(2, 512), (4, 32)], ids=["config2_dims_512", "decode_32"])
def test_noalloc_forward_replays_in_a_hip_graph(cuda, orc, cfg, T):
    # The documented use: a caller under HIP graph capture.  One eager call
    # first (the per-device scratch lookup and the kernels' one-time launch
    # attributes happen outside the capture), then the call captured into a
    # graph, then three replays, each after an eager call with fewer tokens
    # that overwrites the scratch and a host synchronisation.  Every replay is
    # bit-identical to the engine forward and within 2e-2 of the oracle.
    from conftest import rel_err

    inp = synth.config_inputs(cfg, T=T)
    say(f"case: noalloc graph capture cfg {cfg} T {T} ({inp.dtype})")
    eng = moe.MoEEngine(inp.d, inp.f, inp.E, inp.k, inp.n_shared, inp.dtype, max_tokens=T)
    eng.upload(inp.w_router, inp.router_bias, inp.gate, inp.up, inp.down)
    gu, dn = packed_weights(inp)
    wr, rb = dev(inp.w_router), dev(inp.router_bias)
    x = dev(inp.x, inp.dtype)
    ref = eng.forward(x).clone()
    want = orc.moe_forward(inp)["out"]
    out = torch.empty_like(ref)
    assert noalloc_forward(inp, x, wr, rb, gu, dn, out) == L.PRICHS_OK, L.last_error()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = noalloc_forward(inp, x, wr, rb, gu, dn, out)
    assert rc == L.PRICHS_OK, L.last_error()
    xs = x[: max(1, T // 3)].contiguous()
    other = torch.empty((xs.shape[0], inp.d), dtype=ref.dtype, device="cuda")
    for rep in range(3):
        out.fill_(float("nan"))
        assert noalloc_forward(inp, xs, wr, rb, gu, dn, other) == L.PRICHS_OK, L.last_error()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), rep
        err = rel_err(out.float().cpu().numpy(), want)
        assert err <= 2e-2, (rep, err)
        say(f"  replay {rep}: bit-identical to the engine, rel err {err:.2e} against the oracle")
    del graph
    eng.close()
