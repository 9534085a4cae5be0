"""GPU parity of the MoE hot path against the CPU oracle, through the C ABI.

Bars (written in each test):
* routing (logits, selected experts) and the permutation: bit-exact;
* gate weights: within 1e-6 relative (GPU expf vs glibc expf);
* fp32 configurations: max |gpu - ref| / max |ref| <= 1e-4;
* bf16 configurations: max |gpu - ref| / max |ref| <= 2e-2.
"""
import numpy as np
import pytest
import torch

from conftest import rel_err, row_rel_err
from prichs_amd import _lib as L
from prichs_amd import moe, ops, synth

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


# ----------------------------------------------------------------- router --
@pytest.mark.parametrize("cfg", [1, 2, 3, 4])
def test_router_bit_exact(cuda, orc, cfg):
    over = {"T": 4096} if cfg == 3 else {}
    inp = synth.config_inputs(cfg, **over)
    say("router", cfg, inp.T, inp.d)
    logits, idx, w, _ = ops.router_topk(dev(inp.x, inp.dtype), dev(inp.w_router),
                                        dev(inp.router_bias), inp.k)
    rl, rs, rw = orc.route(inp.x, inp.w_router, inp.router_bias, inp.k)
    np.testing.assert_array_equal(host(logits).view(np.uint32), rl.view(np.uint32))
    np.testing.assert_array_equal(host(idx), rs)
    assert rel_err(host(w), rw) <= 1e-6


# Staged kernel (d % 8 == 0; whole and partial K chunks, 1..64 lanes per
# token), the simple kernel (d % 8 != 0, or x not 16-byte aligned) and the
# quad-broadcast kernel (5..8 experts, d % 128 == 0; chunk counts below, at
# and above its register ring, ragged T).
@pytest.mark.parametrize("E,k,T,d", [(4, 2, 77, 64), (8, 1, 33, 96), (16, 3, 200, 128),
                                     (64, 8, 129, 40), (3, 3, 5, 8), (1, 1, 9, 16),
                                     (8, 2, 300, 200), (2, 2, 500, 104), (32, 4, 70, 328),
                                     (6, 2, 100, 37), (8, 2, 64, 13), (8, 2, 77, 128),
                                     (6, 2, 100, 384), (5, 3, 33, 256), (8, 2, 1000, 1536),
                                     (7, 1, 3, 640)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_router_shapes(cuda, orc, E, k, T, d, dtype):
    rng = np.random.default_rng(E * 100 + k)
    x = rng.standard_normal((T, d)).astype(np.float32)
    if dtype == "bf16":
        x = synth.round_bf16(x)
    wr = (0.1 * rng.standard_normal((d, E))).astype(np.float32)
    b = (0.05 * rng.standard_normal(E)).astype(np.float32)
    logits, idx, w, _ = ops.router_topk(dev(x, dtype), dev(wr), dev(b), k)
    rl, rs, rw = orc.route(x, wr, b, k)
    np.testing.assert_array_equal(host(logits).view(np.uint32), rl.view(np.uint32))
    np.testing.assert_array_equal(host(idx), rs)
    assert rel_err(host(w), rw) <= 1e-6


def test_router_unaligned_x(cuda, orc):
    # x starts 4 bytes past a 16-byte boundary: the simple kernel serves it.
    T, d, E, k = 40, 64, 8, 2
    rng = np.random.default_rng(5)
    x = rng.standard_normal((T, d)).astype(np.float32)
    wr = (0.1 * rng.standard_normal((d, E))).astype(np.float32)
    b = np.zeros(E, np.float32)
    buf = torch.zeros(T * d + 1, dtype=torch.float32, device="cuda")
    xv = buf[1:].view(T, d)
    xv.copy_(dev(x))
    logits, idx, w, _ = ops.router_topk(xv, dev(wr), dev(b), k)
    rl, rs, rw = orc.route(x, wr, b, k)
    np.testing.assert_array_equal(host(logits).view(np.uint32), rl.view(np.uint32))
    np.testing.assert_array_equal(host(idx), rs)


@pytest.mark.parametrize("d", [16, 128])
def test_router_ties_nan_and_concept_bias(cuda, orc, d):
    T, E, k = 64, 8, 2
    rng = np.random.default_rng(11)
    x = rng.standard_normal((T, d)).astype(np.float32)
    x[:16] = 0.0  # raw logits exactly +0: selection decided by the bias, with ties
    wr = (0.2 * rng.standard_normal((d, E))).astype(np.float32)
    wr_nan = wr.copy()
    wr_nan[3, 5] = np.nan  # every token gets a NaN logit on expert 5
    b = np.array([0.5, 0.5, -0.0, 0.0, 0.5, 0.1, -1, 0.5], np.float32)
    cb = np.array([0.0, 0.0, 0.25], np.float32)
    for w_r in (wr, wr_nan):
        for concept in (None, cb):
            logits, idx, w, _ = ops.router_topk(dev(x), dev(w_r), dev(b), k,
                                                None if concept is None else dev(concept))
            rl, rs, rw = orc.route(x, w_r, b, k, concept_bias=concept)
            np.testing.assert_array_equal(host(logits).view(np.uint32), rl.view(np.uint32))
            np.testing.assert_array_equal(host(idx), rs)
            gw = host(w)
            assert np.array_equal(np.isnan(gw), np.isnan(rw))
            ok = ~np.isnan(rw)
            assert np.abs(gw[ok] - rw[ok]).max() <= 1e-6


# ------------------------------------------------------------ permutation --
@pytest.mark.parametrize("cfg", [1, 2, 3, 4])
def test_permutation_bit_exact(cuda, orc, cfg):
    over = {"T": 16384} if cfg == 3 else {}
    inp = synth.config_inputs(cfg, **over)
    say("permute", cfg, inp.T)
    _, idx, w, bc = ops.router_topk(dev(inp.x, inp.dtype), dev(inp.w_router),
                                    dev(inp.router_bias), inp.k)
    off, rt, rw, tr = ops.permute(idx, w, bc, inp.E)
    _, rs, rgw = orc.route(inp.x, inp.w_router, inp.router_bias, inp.k)
    o_off, o_rt, o_rw, o_tr = orc.bin_tokens(rs, host(w), inp.E)
    T, k = inp.T, inp.k
    np.testing.assert_array_equal(host(off)[: inp.E + 1], o_off)
    assert host(off)[inp.E + 1] == T * k + T
    np.testing.assert_array_equal(host(rt)[: T * k], o_rt)
    np.testing.assert_array_equal(host(rt)[T * k:], np.arange(T))
    np.testing.assert_array_equal(host(rw), o_rw)
    np.testing.assert_array_equal(host(tr), o_tr)


# ------------------------------------------------------------------ GEMMs --
def _stage_inputs(inp):
    x = dev(inp.x, inp.dtype)
    _, idx, w, bc = ops.router_topk(x, dev(inp.w_router), dev(inp.router_bias), inp.k)
    off, rt, rw, tr = ops.permute(idx, w, bc, inp.E)
    order = list(range(inp.n_shared, inp.n_shared + inp.E)) + list(range(inp.n_shared))
    gu = ops.to_device_packed([ops.pack_gate_up(inp.gate[j], inp.up[j], inp.dtype) for j in order],
                              inp.dtype)
    dn = ops.to_device_packed([ops.pack_down(inp.down[j], inp.dtype) for j in order], inp.dtype)
    return x, idx, w, off, rt, tr, gu, dn, order


@pytest.mark.parametrize("cfg", [1, 2, 3, 4])
def test_grouped_gemms_against_oracle(cuda, orc, cfg):
    inp = synth.config_inputs(cfg)
    say("gemm", cfg)
    T, k, E, d, f = inp.T, inp.k, inp.E, inp.d, inp.f
    x, idx, w, off, rt, tr, gu, dn, order = _stage_inputs(inp)
    G, rows = E + inp.n_shared, T * k + T
    act = ops.grouped_gate_up_swiglu(x, rt, off, G, rows, gu, d, f)
    y = ops.grouped_down(act, off, G, rows, dn, d, f)
    h_off, h_rt = host(off), host(rt)
    h_act, h_y = host(act), host(y)
    tol = TOL[inp.dtype]
    rng = np.random.default_rng(cfg)
    # Every row of every group (config 2: 24,576 rows); at config 3 (49,152
    # rows, skewed groups of ~9.8k and ~2.2k rows) the first and last 96 rows
    # of each group -- its first tiles and its ragged last M-tile -- and 192
    # random rows between them.  Each group's rows meet the bar as a whole and
    # row by row.
    for g in range(G):
        r0, r1 = h_off[g], h_off[g + 1]
        if r1 == r0:
            continue
        sel = np.arange(r0, r1)
        if cfg == 3 and len(sel) > 384:
            mid = rng.choice(sel[96:-96], 192, replace=False)
            sel = np.unique(np.concatenate([sel[:96], sel[-96:], mid]))
        j = order[g]
        xr = inp.x[h_rt[sel]]
        ga = orc.matmul_2d(xr, inp.gate[j])
        ua = orc.matmul_2d(xr, inp.up[j])
        a_ref = orc.swiglu(ga, ua)
        assert rel_err(h_act[sel], a_ref) <= tol, ("act", g)
        e_row, worst = row_rel_err(h_act[sel], a_ref)
        assert e_row <= tol, ("act row", g, int(sel[worst]), e_row)
        # down GEMM on the GPU's own act rows isolates the second GEMM's error
        y_ref = orc.matmul_2d(h_act[sel], inp.down[j])
        assert rel_err(h_y[sel], y_ref) <= tol, ("y", g)
        e_row, worst = row_rel_err(h_y[sel], y_ref)
        assert e_row <= tol, ("y row", g, int(sel[worst]), e_row)
        say(f"  group {g}: {r1 - r0} rows, {len(sel)} checked")


# The tiled gate/up kernel writes 16 bytes per lane when the activations are
# 16-byte aligned and 8 bytes otherwise: an output 8 bytes off alignment must
# get the same bits (groups over 64 rows, so not the skinny kernel).
def test_gate_up_unaligned_output_bit_identical(cuda):
    inp = synth.make_moe_inputs(512, 256, 192, E=8, k=2, dtype="bf16", seed=3)
    x, idx, w, off, rt, tr, gu, dn, order = _stage_inputs(inp)
    G, rows = inp.E + inp.n_shared, inp.T * inp.k + inp.T
    assert int(np.diff(host(off)[: G + 1]).max()) > 64
    say("gate/up unaligned output", rows)
    act = ops.grouped_gate_up_swiglu(x, rt, off, G, rows, gu, inp.d, inp.f)
    flat = torch.zeros(rows * inp.f + 4, dtype=torch.bfloat16, device="cuda")
    view = flat[4:].view(rows, inp.f)  # data 8 bytes past a 16-byte boundary
    assert view.data_ptr() % 16 == 8
    ops.grouped_gate_up_swiglu(x, rt, off, G, rows, gu, inp.d, inp.f, out=view)
    assert torch.equal(act.view(torch.int16), view.view(torch.int16))
    assert int(flat[:4].view(torch.int16).abs().sum()) == 0  # nothing written before it


# Decode-sized groups (every group <= 64 rows) take the skinny weight-streaming
# kernel: empty groups, one 16-row MFMA tile, two tiles, two 32-row M-tiles;
# K with 8, 4 and 2 K-steps per chunk (K % 256, % 128, % 64).
@pytest.mark.parametrize("d,f,counts", [(1536, 1280, [0, 40, 3, 0, 16, 5]),
                                        (320, 384, [17, 1, 0, 32, 14]),
                                        (256, 192, [64]), (1536, 1280, [1, 0, 0, 0, 0, 0, 0, 0, 1])])
def test_skinny_grouped_gemms(cuda, orc, d, f, counts):
    rng = np.random.default_rng(d + f + len(counts))
    G, rows = len(counts), sum(counts)
    Tx = 100
    x = synth.round_bf16(rng.standard_normal((Tx, d)))
    gate = [synth.round_bf16(0.03 * rng.standard_normal((d, f))) for _ in range(G)]
    up = [synth.round_bf16(0.03 * rng.standard_normal((d, f))) for _ in range(G)]
    down = [synth.round_bf16(0.03 * rng.standard_normal((f, d))) for _ in range(G)]
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    row_token = rng.integers(0, Tx, rows).astype(np.int32)
    gu = ops.to_device_packed([ops.pack_gate_up(gate[g], up[g], "bf16") for g in range(G)], "bf16")
    dn = ops.to_device_packed([ops.pack_down(down[g], "bf16") for g in range(G)], "bf16")
    off_d = torch.from_numpy(offsets).to("cuda")
    rt_d = torch.from_numpy(row_token).to("cuda")
    say("skinny", d, f, counts)
    act = ops.grouped_gate_up_swiglu(dev(x, "bf16"), rt_d, off_d, G, rows, gu, d, f)
    y = ops.grouped_down(act, off_d, G, rows, dn, d, f)
    h_act, h_y = host(act), host(y)
    for g in range(G):
        r0, r1 = offsets[g], offsets[g + 1]
        if r1 == r0:
            continue
        xr = x[row_token[r0:r1]]
        a_ref = orc.swiglu(orc.matmul_2d(xr, gate[g]), orc.matmul_2d(xr, up[g]))
        assert rel_err(h_act[r0:r1], a_ref) <= 2e-2, ("act", g)
        assert rel_err(h_y[r0:r1], orc.matmul_2d(h_act[r0:r1], down[g])) <= 2e-2, ("y", g)


@pytest.mark.parametrize("T", [1, 17, 33, 64])
def test_moe_layer_decode_shapes(cuda, orc, T):
    # The engine bounds every group by T, so these take the skinny kernels.
    inp = synth.config_inputs(4, T=T)
    say("layer decode", T)
    layer = moe.MoELayer.from_inputs(inp)
    out, stash = layer.forward_train(inp.x)
    r = orc.moe_forward(inp)
    np.testing.assert_array_equal(stash.selected_experts, r["sel"])
    np.testing.assert_array_equal(stash.row_token, r["row_token"])
    assert rel_err(out, r["out"]) <= TOL["bf16"]
    # Up to 32 tokens the router's single workgroup writes the permutation
    # itself; every permutation output equals the separate permute kernel's.
    _, idx, w, bc = ops.router_topk(dev(inp.x, inp.dtype), dev(inp.w_router),
                                    dev(inp.router_bias), inp.k)
    off, rt, rw, tr = ops.permute(idx, w, bc, inp.E)
    h = layer.engine.stash()
    np.testing.assert_array_equal(host(h["offsets"]), host(off))
    np.testing.assert_array_equal(host(h["row_token"]), host(rt))
    np.testing.assert_array_equal(host(h["row_weight"]).view(np.uint32), host(rw).view(np.uint32))
    np.testing.assert_array_equal(host(h["token_row"]), host(tr))
    layer.engine.close()


def test_aux_free_bias_update_on_device(cuda, orc):
    # moe.rs:228-245 driven as model.rs:1541-1547 drives it, on device; then the
    # next forward routes with the new bias exactly as the oracle does.
    inp = synth.config_inputs(2, T=2048)
    layer = moe.MoELayer.from_inputs(inp)
    _, stash = layer.forward_train(inp.x)
    bias0 = layer.router_bias.copy()
    counts = np.bincount(stash.selected_experts.reshape(-1), minlength=inp.E)
    layer.update_aux_free_bias_on_device(0.001)
    expect = orc.update_aux_free_bias(bias0, counts, inp.k, inp.T, 0.001)
    np.testing.assert_array_equal(layer.router_bias.view(np.uint32), expect.view(np.uint32))
    assert not np.array_equal(expect, bias0)
    _, stash2 = layer.forward_train(inp.x)
    _, sel2, _ = orc.route(inp.x, inp.w_router, expect, inp.k)
    np.testing.assert_array_equal(stash2.selected_experts, sel2)
    # After a forward of zero tokens the update is a no-op (total_tokens == 0).
    layer.engine.forward(torch.empty((0, inp.d), dtype=torch.bfloat16, device="cuda"))
    layer.update_aux_free_bias_on_device(0.001)
    np.testing.assert_array_equal(layer.router_bias, expect)
    layer.engine.close()


@pytest.mark.parametrize("E,k", [(6, 1), (5, 3), (7, 2)])
def test_decode_fused_permutation_other_experts(cuda, orc, E, k):
    # The quad router (5-8 experts) writes the permutation itself when one
    # workgroup covers the batch; with fewer than 8 experts and k != 2 its
    # outputs equal the separate permute kernel's, and the layer matches the
    # oracle (routing bit-exact, outputs within 2e-2).
    inp = synth.make_moe_inputs(T=17, d=256, f=128, E=E, k=k, dtype="bf16", seed=E * 10 + k,
                                name=f"decode-E{E}-k{k}")
    say("fused permutation", E, k)
    assert ops.router_num_blocks(inp.T, E) == 1
    layer = moe.MoELayer.from_inputs(inp)
    out, stash = layer.forward_train(inp.x)
    r = orc.moe_forward(inp)
    np.testing.assert_array_equal(stash.selected_experts, r["sel"])
    np.testing.assert_array_equal(stash.row_token, r["row_token"])
    assert rel_err(out, r["out"]) <= TOL["bf16"]
    _, idx, w, bc = ops.router_topk(dev(inp.x, inp.dtype), dev(inp.w_router),
                                    dev(inp.router_bias), inp.k)
    off, rt, rw, tr = ops.permute(idx, w, bc, inp.E)
    h = layer.engine.stash()
    np.testing.assert_array_equal(host(h["offsets"]), host(off))
    np.testing.assert_array_equal(host(h["row_token"]), host(rt))
    np.testing.assert_array_equal(host(h["row_weight"]).view(np.uint32), host(rw).view(np.uint32))
    np.testing.assert_array_equal(host(h["token_row"]), host(tr))
    layer.engine.close()


# ------------------------------------------------ engine permutation reuse --
@pytest.mark.parametrize("d,Ts", [(1536, [8192, 1000, 33, 8192, 4096]), (128, [8192, 700])],
                         ids=["config2_dims", "d128"])
def test_engine_permutation_across_batch_sizes(cuda, d, Ts):
    # Consecutive forwards of different sizes on one engine (different router
    # workgroup counts, so different histogram layouts in the reused
    # buffers) must each give exactly the standalone router + permutation
    # kernels' outputs.
    E, k, f = 8, 2, 128
    inp = synth.make_moe_inputs(T=max(Ts), d=d, f=f, E=E, k=k, dtype="bf16", seed=d,
                                name=f"perm-d{d}")
    say("engine permutation across batch sizes", d, Ts)
    eng = moe.MoEEngine(d, f, E, k, 1, "bf16", max_tokens=max(Ts))
    eng.upload(inp.w_router, inp.router_bias, inp.gate, inp.up, inp.down)
    x = dev(inp.x, "bf16")
    wr, rb = dev(inp.w_router), dev(inp.router_bias)
    for T in Ts:
        xs = x[:T].contiguous()
        eng.forward(xs)
        st = eng.stash()
        _, idx, w, bc = ops.router_topk(xs, wr, rb, k)
        off, rt, rw, tr = ops.permute(idx, w, bc, E)
        torch.cuda.synchronize()
        assert torch.equal(st["selected_experts"].view(-1), idx.view(-1)), T
        assert torch.equal(st["offsets"], off), T
        assert torch.equal(st["row_token"], rt), T
        assert torch.equal(st["row_weight"].view(torch.int32), rw.view(torch.int32)), T
        assert torch.equal(st["token_row"], tr), T
    eng.close()


# ------------------------------------------------------------ decode path --
@pytest.mark.parametrize("T,E,k,concept", [(32, 8, 2, False), (17, 8, 2, True), (1, 8, 2, False),
                                           (5, 6, 3, False), (32, 5, 1, True)],
                         ids=["T32", "T17_concept", "T1", "T5_E6_k3", "T32_E5_k1_concept"])
def test_decode_path_bit_identical_to_routed_path(cuda, orc, T, E, k, concept):
    # When one router workgroup covers the batch, the engine runs the router
    # (and the permutation) inside a gate/up launch that covers every token
    # of every expert, and the down GEMM gathers the routed rows.  An engine
    # with the backward enabled keeps the routed stages (router, permutation,
    # routed gate/up, down).  Routing, the permutation, the stash's act and y
    # rows and the output are the same bits on both; the output is within
    # 2e-2 of the oracle.
    d, f = (1536, 1280) if E == 8 and k == 2 else (256, 128)
    inp = synth.make_moe_inputs(T=T, d=d, f=f, E=E, k=k, dtype="bf16", seed=100 + T + E,
                                name=f"decode-T{T}-E{E}-k{k}")
    say("decode vs routed", T, E, k, concept)
    cb = None
    if concept:
        cb_np = np.zeros(E, np.float32)
        cb_np[E - 1] = 0.5
        cb = dev(cb_np)
    x = dev(inp.x, "bf16")
    outs, outs32, stashes = [], [], []
    for backward in (False, True):
        eng = moe.MoEEngine(d, f, E, k, 1, "bf16", max_tokens=max(T, 32))
        if backward:
            eng.enable_backward()
        eng.upload(inp.w_router, inp.router_bias, inp.gate, inp.up, inp.down)
        outs.append(eng.forward(x, concept_bias=cb).clone())
        outs32.append(eng.forward(x, concept_bias=cb, out_dtype=torch.float32).clone())
        stashes.append(eng.stash())
        if not backward:
            # A misaligned output takes the combine's one-column-per-thread
            # kernel instead of the 8-column one: same bits, bf16 and f32.
            for dt, ref in ((torch.bfloat16, outs[0]), (torch.float32, outs32[0])):
                buf = torch.empty(T * d + 8, dtype=dt, device="cuda")
                mis = buf[1:1 + T * d].view(T, d)
                eng.forward(x, concept_bias=cb, out=mis)
                iv = torch.int16 if dt == torch.bfloat16 else torch.int32
                assert torch.equal(mis.view(iv), ref.view(iv)), dt
        eng.close()
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    assert torch.equal(outs32[0].view(torch.int32), outs32[1].view(torch.int32))
    for name in ("router_logits", "selected_experts", "gating_weights", "offsets", "row_token",
                 "row_weight", "token_row", "act", "y"):
        a, b = stashes[0][name], stashes[1][name]
        a, b = (a.view(torch.int16), b.view(torch.int16)) if a.dtype == torch.bfloat16 else (a, b)
        assert torch.equal(a, b), name
    r = orc.moe_forward(inp, concept_bias=None if cb is None else host(cb))
    np.testing.assert_array_equal(host(stashes[0]["selected_experts"]), r["sel"])
    np.testing.assert_array_equal(host(stashes[0]["row_token"])[:T * k], r["row_token"])
    np.testing.assert_array_equal(host(stashes[0]["offsets"])[:E + 1], r["offsets"])
    e_row, worst = row_rel_err(host(outs[0].float()), r["out"])
    assert e_row <= TOL["bf16"], (worst, e_row)


# ---------------------------------------------------- graph capture --
def test_engine_forward_replays_in_a_hip_graph(cuda):
    # The engine forward captured into a graph (router, permutation, gate/up,
    # down, combine: no allocation, no memset node, no host synchronisation)
    # and replayed three times, each after an eager forward of another size
    # (which rewrites every intermediate) and a host synchronisation: every
    # replay is bit-identical to the eager result.
    inp = synth.config_inputs(2, T=4096)
    say("case: engine forward graph replay T 4096")
    eng = moe.MoEEngine(inp.d, inp.f, inp.E, inp.k, 1, "bf16", max_tokens=4096)
    eng.upload(inp.w_router, inp.router_bias, inp.gate, inp.up, inp.down)
    x = dev(inp.x, "bf16")
    out = torch.empty((4096, inp.d), dtype=torch.bfloat16, device="cuda")
    eng.forward(x, out=out)
    torch.cuda.synchronize()
    ref = out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        eng.forward(x, out=out)
    xs = x[:1500].contiguous()
    for rep in range(3):
        out.fill_(float("nan"))
        eng.forward(xs)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), rep
        say(f"  replay {rep}: bit-identical")
    del graph
    eng.close()


def test_decode_forward_replays_in_a_hip_graph(cuda):
    # The decode path (router and permutation inside the gate/up launch, the
    # down GEMM gathering the routed rows) captured at T = 32 and replayed
    # three times, each after eager forwards of other sizes on both paths:
    # every replay is bit-identical.
    inp = synth.config_inputs(4)
    T = inp.T
    say("case: decode forward graph replay T", T)
    eng = moe.MoEEngine(inp.d, inp.f, inp.E, inp.k, 1, "bf16", max_tokens=256)
    eng.upload(inp.w_router, inp.router_bias, inp.gate, inp.up, inp.down)
    x = dev(inp.x, "bf16")
    out = torch.empty((T, inp.d), dtype=torch.bfloat16, device="cuda")
    eng.forward(x, out=out)
    torch.cuda.synchronize()
    ref = out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        eng.forward(x, out=out)
    x17 = x[:17].contiguous()
    x_big = torch.cat([x] * 8).contiguous()
    for rep in range(3):
        out.fill_(float("nan"))
        eng.forward(x17)
        eng.forward(x_big)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), rep
        say(f"  replay {rep}: bit-identical")
    del graph
    eng.close()


# ------------------------------------------------------------- full layer --
@pytest.mark.parametrize("cfg", [1, 2, 4])
def test_moe_layer_full_against_oracle(cuda, orc, cfg):
    inp = synth.config_inputs(cfg)
    say("layer", cfg, inp.T)
    layer = moe.MoELayer.from_inputs(inp)
    out, stash = layer.forward_train(inp.x)
    r = orc.moe_forward(inp)
    np.testing.assert_array_equal(stash.selected_experts, r["sel"])
    np.testing.assert_array_equal(stash.router_logits.view(np.uint32), r["logits"].view(np.uint32))
    np.testing.assert_array_equal(stash.expert_offsets, r["offsets"])
    np.testing.assert_array_equal(stash.row_token, r["row_token"])
    assert rel_err(stash.gating_weights, r["gw"]) <= 1e-6
    assert rel_err(out, r["out"]) <= TOL[inp.dtype]
    # The same bar on every token's row on its own.
    e_row, worst = row_rel_err(out, r["out"])
    say(f"  worst row {worst}: rel err {e_row:.3e} (experts {r['sel'][worst].tolist()})")
    assert e_row <= TOL[inp.dtype], (worst, e_row)
    layer.engine.close()


def test_moe_layer_skewed_config3_full(cuda, orc):
    # Full size (16384 tokens, ~60% of rows on experts 0-1): routing, the
    # permutation and the output of every token against the oracle.
    inp = synth.config_inputs(3)
    say("layer skew", inp.T)
    layer = moe.MoELayer.from_inputs(inp)
    out, stash = layer.forward_train(inp.x)
    _, rs, _ = orc.route(inp.x, inp.w_router, inp.router_bias, inp.k)
    np.testing.assert_array_equal(stash.selected_experts, rs)
    cnt = np.bincount(rs.reshape(-1), minlength=inp.E)
    assert 0.59 <= (cnt[0] + cnt[1]) / rs.size <= 0.61
    o_off, o_rt, _, _ = orc.bin_tokens(rs, stash.gating_weights, inp.E)
    np.testing.assert_array_equal(stash.expert_offsets, o_off)
    np.testing.assert_array_equal(stash.row_token, o_rt)
    r = orc.moe_forward(inp)
    np.testing.assert_array_equal(stash.row_token, r["row_token"])
    assert rel_err(out, r["out"]) <= TOL["bf16"]
    e_row, worst = row_rel_err(out, r["out"])
    say(f"  worst row {worst}: rel err {e_row:.3e} (experts {r['sel'][worst].tolist()})")
    assert e_row <= TOL["bf16"], (worst, e_row)
    # Per token group: the bar on the tokens routed to each expert alone
    # (experts 0 and 1 hold ~9.8k tokens each, the rest ~2.2k).
    for e in range(inp.E):
        tok = np.nonzero((rs == e).any(axis=1))[0]
        e_g = rel_err(out[tok], r["out"][tok])
        assert e_g <= TOL["bf16"], (e, len(tok), e_g)
    layer.engine.close()


def test_moe_row_space_past_2_32_elements(cuda, orc):
    # A configuration-2 layer over T = 1.2M tokens: the down GEMM's A operand
    # (act, T (k + 1) x f = 4.6e9 elements) and y (5.5e9) pass 2^32 elements,
    # so the shared rows of the last ~245k tokens sit past any 32-bit element
    # offset.  Rows are independent (test_moe_rows_are_independent), so the
    # first and last tokens are checked against the oracle on those tokens
    # alone: routing bit-exact, outputs within 2e-2.
    T = 1_200_000
    inp = synth.config_inputs(2, T=64)
    say("large row space", T)
    gen = torch.Generator(device="cuda").manual_seed(7)
    x = torch.randn((T, inp.d), generator=gen, device="cuda").to(torch.bfloat16)
    eng = moe.MoEEngine(inp.d, inp.f, inp.E, inp.k, 1, "bf16", max_tokens=T)
    eng.upload(inp.w_router, inp.router_bias, inp.gate, inp.up, inp.down)
    out = eng.forward(x)
    assert (T * (inp.k + 1) - 1) * inp.f >= 2**32
    rows = torch.cat([torch.arange(0, 64), torch.arange(T - 256, T)]).cuda()
    got = out[rows].float().cpu().numpy()
    sel = eng.stash(["selected_experts"])["selected_experts"][rows].cpu().numpy()
    sub = synth.MoEInputs(**{**inp.__dict__, "x": x[rows].float().cpu().numpy(), "T": len(rows)})
    r = orc.moe_forward(sub)
    np.testing.assert_array_equal(sel, r["sel"])
    assert rel_err(got, r["out"]) <= TOL["bf16"]
    del x, out
    eng.close()


def test_moe_forward_deterministic_and_ragged(cuda, orc):
    inp = synth.config_inputs(2, T=1000)  # ragged: not a multiple of any tile
    eng = moe.MoEEngine(inp.d, inp.f, inp.E, inp.k, 1, "bf16", max_tokens=inp.T)
    eng.upload(inp.w_router, inp.router_bias, inp.gate, inp.up, inp.down)
    x = dev(inp.x, "bf16")
    o1 = eng.forward(x, out_dtype=torch.float32)
    o2 = eng.forward(x, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)  # no atomics: bitwise reproducible
    r = orc.moe_forward(inp)
    assert rel_err(host(o1), r["out"]) <= TOL["bf16"]
    # smaller batches reuse the same workspace; T = 1 and an empty batch
    for T in (1, 17, 0):
        sub = synth.MoEInputs(**{**inp.__dict__, "x": inp.x[:T], "T": T})
        o = eng.forward(dev(inp.x[:T], "bf16"), out_dtype=torch.float32)
        if T:
            assert rel_err(host(o), orc.moe_forward(sub)["out"]) <= TOL["bf16"]
    # capacity errors are reported, not faulted
    with pytest.raises(L.PrichsError) as e:
        eng.forward(dev(np.zeros((inp.T + 1, inp.d), np.float32), "bf16"))
    assert e.value.status == L.PRICHS_ERR_CAPACITY
    eng.close()


def test_moe_bf16_output_and_aux_bias(cuda, orc):
    inp = synth.config_inputs(4)
    layer = moe.MoELayer.from_inputs(inp)
    x = dev(inp.x, "bf16")
    ob = layer.engine.forward(x, out_dtype=torch.bfloat16)
    r = orc.moe_forward(inp)
    assert rel_err(host(ob), r["out"]) <= TOL["bf16"]
    # aux-loss-free bias update (moe.rs:228-245) changes routing on the device.
    counts = np.bincount(r["sel"].reshape(-1), minlength=inp.E)
    layer.update_aux_free_bias(counts, inp.T, 5.0)
    out2, st2 = layer.forward_train(inp.x)
    inp2 = synth.MoEInputs(**{**inp.__dict__, "router_bias": layer.router_bias.copy()})
    r2 = orc.moe_forward(inp2)
    np.testing.assert_array_equal(st2.selected_experts, r2["sel"])
    assert rel_err(out2, r2["out"]) <= TOL["bf16"]
    layer.engine.close()


def test_engine_stage_timing(cuda):
    inp = synth.config_inputs(4)
    eng = moe.MoEEngine(inp.d, inp.f, inp.E, inp.k, 1, "bf16", max_tokens=inp.T)
    eng.upload(inp.w_router, inp.router_bias, inp.gate, inp.up, inp.down)
    eng.set_timing(3)
    for _ in range(5):
        eng.forward(dev(inp.x, "bf16"))
    ms = eng.stage_ms()
    assert ms["n"] == 3
    assert all(v >= 0 for v in ms.values())
    assert ms["total"] >= max(ms["gate_up"], ms["down"])
    eng.close()
