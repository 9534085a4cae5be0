"""Engines loaded from a reference weight file (PRICHS02,
crates/prichs-model/src/model.rs:1648-1736) on the GPU.

An engine uploaded from block `layer` of a file must equal, bit for bit, an
engine uploaded directly with the same weights: block 0 of each file holds
other weights, so a wrong index map or a swapped tensor shows up.  The
checkpointed MoE engine is also checked against the CPU oracle (routing
bit-exact, output <= 2e-2 in bf16).
"""
import numpy as np
import pytest
import torch

from conftest import rel_err
from prichs_amd import _lib as L
from prichs_amd import block, checkpoint as ck, moe, synth

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def _block_tensors(d, kvw, m: synth.MoEInputs, rng, attn=None):
    """One block in the order of get_parameter_tensors (model.rs:318-333)."""
    if attn is None:
        attn = dict(input_norm=1 + 0.02 * rng.standard_normal(d), q=0.02 * rng.standard_normal((d, d)),
                    k=0.02 * rng.standard_normal((d, kvw)), v=0.02 * rng.standard_normal((d, kvw)),
                    o=0.02 * rng.standard_normal((d, d)), post=1 + 0.02 * rng.standard_normal(d))
    t = [attn["input_norm"], attn["q"], attn["k"], attn["v"], attn["o"], attn["post"], m.w_router]
    for g, u, dn in zip(m.gate, m.up, m.down):  # shared expert first, then routed 0..E-1
        t += [g, u, dn]
    return t


def _write(path, d, blocks, vocab=16, seed=0):
    rng = np.random.default_rng(seed)
    tensors = [0.02 * rng.standard_normal((vocab, d)), np.ones(d)]
    for b in blocks:
        tensors += b
    ck.write_prichs02(path, 123, 1.25, [np.asarray(t, np.float32) for t in tensors])


def test_moe_engine_from_checkpoint(cuda, orc, tmp_path):
    d, f, E, k, T = 128, 128, 8, 2, 96
    inp = synth.make_moe_inputs(T, d, f, E, k, dtype="bf16", seed=5, name="ckpt")
    decoy = synth.make_moe_inputs(8, d, f, E, k, dtype="bf16", seed=6, name="decoy")
    rng = np.random.default_rng(1)
    path = tmp_path / "moe.prichs"
    _write(path, d, [_block_tensors(d, 64, decoy, rng), _block_tensors(d, 64, inp, rng)])
    say("moe from checkpoint", path.stat().st_size)
    direct = moe.MoEEngine(d, f, E, k, max_tokens=T)
    direct.upload(inp.w_router, inp.router_bias, inp.gate, inp.up, inp.down)
    loaded = moe.MoEEngine(d, f, E, k, max_tokens=T)
    with ck.Checkpoint(path) as c:
        assert (c.step, c.loss, c.n_params) == (123, 1.25, 2 + 2 * (10 + 3 * E))
        loaded.upload_checkpoint(c, 1, router_bias=inp.router_bias)
        # Block 2 is not in the file; a wrong f and a shared-less engine are refused.
        with pytest.raises(L.PrichsError) as e:
            loaded.upload_checkpoint(c, 2)
        assert e.value.status == L.PRICHS_ERR_INVALID_ARGUMENT
        wrong_f = moe.MoEEngine(d, 192, E, k, max_tokens=T)
        with pytest.raises(L.PrichsError) as e:
            wrong_f.upload_checkpoint(c, 1)
        assert e.value.status == L.PRICHS_ERR_INVALID_ARGUMENT and "expects" in e.value.message
        no_shared = moe.MoEEngine(d, f, E, k, n_shared=0, max_tokens=T)
        with pytest.raises(L.PrichsError) as e:
            no_shared.upload_checkpoint(c, 1)
        assert e.value.status == L.PRICHS_ERR_UNSUPPORTED
        for eng in (wrong_f, no_shared):
            eng.close()
    x = torch.from_numpy(inp.x).to("cuda").to(torch.bfloat16)
    oa = direct.forward(x, out_dtype=torch.float32)
    ob = loaded.forward(x, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(oa, ob)
    r = orc.moe_forward(inp)
    sel = loaded.stash()["selected_experts"].cpu().numpy()
    np.testing.assert_array_equal(sel, r["sel"])
    assert rel_err(ob.cpu().numpy(), r["out"]) <= 2e-2
    direct.close()
    loaded.close()


def test_block_engine_from_checkpoint(cuda, tmp_path):
    inp = synth.make_block_inputs(batch=1, seq_len=64, d=256, n_heads=2, n_kv_heads=1, f=128,
                                  name="ckpt-block")
    m = inp.moe
    attn = dict(input_norm=inp.input_norm, q=inp.wq, k=inp.wk, v=inp.wv, o=inp.wo,
                post=inp.post_norm)
    decoy = synth.make_moe_inputs(8, inp.d, m.f, m.E, m.k, dtype="bf16", seed=9, name="decoy")
    rng = np.random.default_rng(2)
    kvw = inp.n_kv_heads * inp.head_dim
    path = tmp_path / "block.prichs"
    _write(path, inp.d, [_block_tensors(inp.d, kvw, decoy, rng), _block_tensors(inp.d, kvw, m, rng, attn)])
    say("block from checkpoint", path.stat().st_size)
    mk = lambda: block.BlockEngine(inp.d, inp.n_heads, inp.n_kv_heads, m.f, m.E, m.k,  # noqa: E731
                                   max_tokens=64, max_seq_len=1024, rope_theta=inp.rope_theta,
                                   eps=inp.eps)
    direct, loaded = mk(), mk()
    direct.upload(inp.input_norm, inp.post_norm, inp.wq, inp.wk, inp.wv, inp.wo, m.w_router,
                  m.router_bias, m.gate, m.up, m.down)
    with ck.Checkpoint(path) as c:
        loaded.upload_checkpoint(c, 1, router_bias=m.router_bias)
    x = torch.from_numpy(inp.x).to("cuda").to(torch.bfloat16)
    oa = direct.forward(x, 1, 64, out_dtype=torch.float32)
    ob = loaded.forward(x, 1, 64, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(oa, ob)
    direct.close()
    loaded.close()
