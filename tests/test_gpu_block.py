"""GPU parity of the PrichsBlock path (config 5) against the CPU oracle and
float64 references, through the C ABI.

Bars (written in each test):
* dense GEMM (bf16 in/out, fp32 accumulate): max |gpu - ref| / max |ref| <= 1e-2;
* residual add: bit-exact (one f32 addition, then the output rounding);
* attention kernel (bf16 q/k/v/out, bf16 probabilities): <= 2e-2 against a
  float64 softmax attention of the same bf16 inputs;
* whole block (bf16): each sub-layer <= 2e-2 on its own GPU input (MoE routing
  bit-exact); block output <= 2e-2 on tokens routed as the f32 oracle routes
  them, with at most 2% of tokens flipped by bf16 rounding at near-ties.
"""
import numpy as np
import pytest
import torch

from conftest import rel_err, row_rel_err
from prichs_amd import block, ops, synth

pytestmark = pytest.mark.gpu


def dev(a, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to("cuda").to(dtype)


def host(t):
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


def say(*a):
    print(*a, flush=True)


@pytest.mark.parametrize("M,K,N", [(300, 256, 320), (1, 64, 64), (4096, 1536, 2304)])
def test_dense_gemm(cuda, orc, M, K, N):
    rng = np.random.default_rng(M + K + N)
    a = synth.round_bf16(rng.standard_normal((M, K)))
    w = synth.round_bf16(0.05 * rng.standard_normal((K, N)))
    wp = ops.to_device_packed([ops.pack_weight(w, "bf16")], "bf16")
    c = ops.gemm(dev(a), wp, N)
    ref = orc.matmul_2d(a, w)
    assert rel_err(host(c), ref) <= 1e-2
    # Output into a column slice of a wider buffer (ldc > N).
    wide = torch.zeros((M, N + 64), dtype=torch.bfloat16, device="cuda")
    ops.gemm(dev(a), wp, N, out=wide[:, 32:32 + N])
    hw = host(wide)
    np.testing.assert_array_equal(hw[:, 32:32 + N], host(c))
    assert not hw[:, :32].any() and not hw[:, 32 + N:].any()


def _tile_times(tiles, grid, split):
    full, tail = divmod(tiles, grid)
    if tail == 0:
        return full
    return full + (0.6 if split and 2 * tail <= grid else 1.0)


def _dense_cfg(M, N, cus):
    """Mirror of the dense launcher's choice: ("square" | "wide" | "tall", tail
    split).  Square = 256 x 256 tiles on a grid of min(2 (M/256 + 1) N/256,
    CUs) whose last partial round of t tiles is split into half-width tiles
    when 2 t fits the grid; wide = 128 x 384 tiles (N a multiple of 384) on
    min((M/128 + 1) N/384, CUs), never split, each 0.75 of a square tile's
    work at 0.96 of its rate; tall = 256 x 288 tiles (N a multiple of 288) on
    min((M/256 + 1) N/288, CUs), never split, 1.125 of a square tile's work.
    The fastest estimate wins (ties keep the earlier shape)."""
    sq_tiles = -(-M // 256) * (N // 256)
    sq_grid = min(2 * (M // 256 + 1) * (N // 256), cus)
    tail = sq_tiles % sq_grid
    split = 0 < tail and 2 * tail <= sq_grid
    best, cfg = _tile_times(sq_tiles, sq_grid, True), ("square", split)
    if N % 384 == 0:
        wd_tiles = -(-M // 128) * (N // 384)
        wd_grid = min((M // 128 + 1) * (N // 384), cus)
        t = _tile_times(wd_tiles, wd_grid, False) * 0.75 / 0.96
        if t < best:
            best, cfg = t, ("wide", False)
    if N % 288 == 0:
        tl_tiles = -(-M // 256) * (N // 288)
        tl_grid = min((M // 256 + 1) * (N // 288), cus)
        t = _tile_times(tl_tiles, tl_grid, False) * 1.125
        if t < best:
            best, cfg = t, ("tall", False)
    return cfg


def test_gemm_tail_round_halves_bit_identical(cuda):
    """The last partial round of the down / dense GEMM runs as half-width
    tiles, and some dense launches run as 128 x 384 tiles: every output
    element is the same MFMA chain over K, so rows computed either way are
    bit-identical to the same rows of a launch that computes them as whole
    256 x 256 tiles, and within the 1e-2 bar of float64."""
    K = N = 1536
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    rng = np.random.default_rng(11)
    a = synth.round_bf16(rng.standard_normal((20000, K)))
    w = synth.round_bf16(0.05 * rng.standard_normal((K, N)))
    wp = ops.to_device_packed([ops.pack_weight(w, "bf16")], "bf16")
    assert _dense_cfg(20000, N, cus) == ("square", False)
    whole = host(ops.gemm(dev(a), wp, N))
    seen = set()
    for M in (4096, 8192, 12000, 12288):
        cfg = _dense_cfg(M, N, cus)
        seen.add(cfg)
        say(f"dense gemm M={M}: tiles {cfg[0]}, tail split {cfg[1]} on {cus} CUs")
        c = host(ops.gemm(dev(a[:M]), wp, N))
        np.testing.assert_array_equal(c, whole[:M])
        lo = max(0, M - 2048)  # the tail tiles hold the last M-tiles
        ref = a[lo:M].astype(np.float64) @ w.astype(np.float64)
        assert rel_err(c[lo:], ref) <= 1e-2
    if cus == 256:
        assert ("square", True) in seen and ("wide", False) in seen, seen


def test_dense_gemm_qkv_shape_tiles(cuda, orc):
    """The block's q/k/v projection shape (8192 x 2304, K = 1536) runs as
    256 x 288 tiles on 256 CUs (one round; 18 B blocks per stage dealt
    unevenly over the 8 waves): against the oracle's matmul_2d on row slices,
    and bit-identical to the rows of launches that pick 128 x 384 tiles (4096
    rows) and 256 x 256 tiles with a half-width tail (2048 rows)."""
    M, K, N = 8192, 1536, 2304
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    cfgs = {m: _dense_cfg(m, N, cus)[0] for m in (M, 4096, 2048)}
    say(f"dense gemm {N}x{K}: tiles by rows {cfgs} on {cus} CUs")
    if cus == 256:
        assert cfgs == {M: "tall", 4096: "wide", 2048: "square"}, cfgs
    rng = np.random.default_rng(5)
    a = synth.round_bf16(rng.standard_normal((M, K)))
    w = synth.round_bf16(0.05 * rng.standard_normal((K, N)))
    wp = ops.to_device_packed([ops.pack_weight(w, "bf16")], "bf16")
    c = host(ops.gemm(dev(a), wp, N))
    for lo in (0, 4000, M - 256):
        ref = orc.matmul_2d(a[lo:lo + 256], w)
        assert rel_err(c[lo:lo + 256], ref) <= 1e-2, lo
    for m2 in (4096, 2048):
        np.testing.assert_array_equal(host(ops.gemm(dev(a[:m2]), wp, N)), c[:m2])


def test_residual_add_bit_exact(cuda):
    rng = np.random.default_rng(1)
    a = synth.round_bf16(rng.standard_normal(4096))
    b = synth.round_bf16(rng.standard_normal(4096))
    s = ops.add(dev(a), dev(b), out_dtype=torch.float32)
    np.testing.assert_array_equal(host(s), a + b)  # f32 sum of bf16 values
    s2 = ops.add(dev(a, torch.float32), dev(b), out_dtype=torch.bfloat16)
    np.testing.assert_array_equal(host(s2), synth.round_bf16(a + b))


def _attention_f64(q, k, v, B, S, Hq, Hkv, heads=None, seqs=None):
    """float64 causal GQA attention of [B*S, H*128] rows; returns {(b, h): [S, 128]}."""
    hd = 128
    group = Hq // Hkv
    mask = np.tril(np.ones((S, S), bool))
    out = {}
    for b in (seqs if seqs is not None else range(B)):
        rows = slice(b * S, (b + 1) * S)
        for h in (heads if heads is not None else range(Hq)):
            kv = h // group
            qh = q[rows, h * hd:(h + 1) * hd].astype(np.float64)
            kh = k[rows, kv * hd:(kv + 1) * hd].astype(np.float64)
            vh = v[rows, kv * hd:(kv + 1) * hd].astype(np.float64)
            sc = np.where(mask, qh @ kh.T / np.sqrt(hd), -np.inf)
            p = np.exp(sc - sc.max(1, keepdims=True))
            out[(b, h)] = (p / p.sum(1, keepdims=True)) @ vh
    return out


# GQA groups of 1, 2 and 4 query heads per kv head (1, 2 or 4 heads share a
# workgroup's K/V tiles), ragged and single-row sequences.
@pytest.mark.parametrize("B,S,Hq,Hkv", [(2, 200, 4, 2), (1, 128, 2, 1), (1, 64, 1, 1),
                                        (2, 333, 3, 3), (1, 1, 2, 1), (1, 100, 8, 2),
                                        (2, 257, 4, 1), (1, 31, 12, 3)])
def test_attention_kernel(cuda, B, S, Hq, Hkv):
    rng = np.random.default_rng(B * 1000 + S + Hq)
    hd = 128
    n = (Hq + 2 * Hkv) * hd
    qkv = synth.round_bf16(rng.standard_normal((B * S, n)) * 0.7)
    qkv_d = dev(qkv)
    q = qkv_d[:, :Hq * hd]
    k = qkv_d[:, Hq * hd:(Hq + Hkv) * hd]
    v = qkv_d[:, (Hq + Hkv) * hd:]
    o = host(ops.attention(q, k, v, B, S, Hq, Hkv))
    ref = _attention_f64(qkv[:, :Hq * hd], qkv[:, Hq * hd:(Hq + Hkv) * hd],
                         qkv[:, (Hq + Hkv) * hd:], B, S, Hq, Hkv)
    for (b, h), r in ref.items():
        got = o[b * S:(b + 1) * S, h * hd:(h + 1) * hd]
        assert rel_err(got, r) <= 2e-2, (b, h)


def test_attention_kernel_config5_shape(cuda):
    # 4 sequences x 2048, 12 query heads on 3 kv heads; sampled (b, h) checked.
    B, S, Hq, Hkv, hd = 4, 2048, 12, 3, 128
    rng = np.random.default_rng(55)
    n = (Hq + 2 * Hkv) * hd
    qkv = synth.round_bf16(rng.standard_normal((B * S, n)).astype(np.float32))
    qkv_d = dev(qkv)
    say("attention config5 shape")
    o = host(ops.attention(qkv_d[:, :1536], qkv_d[:, 1536:1920], qkv_d[:, 1920:], B, S, Hq, Hkv))
    ref = _attention_f64(qkv[:, :1536], qkv[:, 1536:1920], qkv[:, 1920:], B, S, Hq, Hkv,
                         heads=[0, 5, 11], seqs=[0, 3])
    for (b, h), r in ref.items():
        assert rel_err(o[b * S:(b + 1) * S, h * hd:(h + 1) * hd], r) <= 2e-2, (b, h)


def _check_block(orc, inp):
    """Each sub-layer against the oracle fed the GPU's own input to it, then the
    block output end to end.  bf16 activations make the GPU's MoE input differ
    from the f32 oracle's in the last bits, which can flip the top-2 choice of
    tokens sitting on a near-tie; such tokens are counted (and bounded), the
    rest must meet the bf16 bar."""
    blk = block.PrichsBlock.from_inputs(inp)
    x = dev(inp.x)
    out = host(blk.engine.forward(x, inp.batch, inp.seq_len, out_dtype=torch.float32))
    st = {n: host(t) if t.dtype != torch.int32 else t.cpu().numpy()
          for n, t in blk.engine.stash().items()}
    r = orc.block_forward(inp)
    # 0. The fused residual add + post-attention norm is bit-identical to an
    #    f32 add of the bf16 operands followed by the stand-alone RMSNorm kernel.
    np.testing.assert_array_equal(st["x1"], synth.round_bf16(inp.x) + st["attn_out"])
    n2_alone, _ = ops.rmsnorm(dev(st["x1"], torch.float32), dev(inp.post_norm, torch.float32),
                              eps=inp.eps, out_dtype=torch.bfloat16, want_rstd=False)
    np.testing.assert_array_equal(st["normed2"], host(n2_alone))
    #    The final residual add rides in the MoE combine: out = x1 + moe_out
    #    (f32 add of the bf16 sub-layer output), bit for bit, in f32 and bf16.
    np.testing.assert_array_equal(out, st["x1"] + st["moe_out"])
    out_bf = host(blk.engine.forward(x, inp.batch, inp.seq_len, out_dtype=torch.bfloat16))
    np.testing.assert_array_equal(out_bf, synth.round_bf16(st["x1"] + st["moe_out"]))
    # 1. attention sub-layer (input: x itself, identical on both sides).
    e_att = rel_err(st["attn_out"], r["attn"])
    # 2. MoE sub-layer on the GPU's own normed2 (bf16 values): routing bit-exact.
    m = inp.moe
    sub = synth.MoEInputs(**{**m.__dict__, "x": st["normed2"], "T": st["normed2"].shape[0]})
    rm = orc.moe_forward(sub)
    np.testing.assert_array_equal(st["selected_experts"], rm["sel"])
    np.testing.assert_array_equal(st["router_logits"].view(np.uint32), rm["logits"].view(np.uint32))
    e_moe = rel_err(st["moe_out"], rm["out"])
    # 3. end to end against the f32 oracle, on tokens routed alike.
    n2_ref = orc.rms_norm(r["x1"], inp.post_norm, inp.eps)
    _, sel_ref, _ = orc.route(n2_ref, m.w_router, m.router_bias, m.k)
    same = (np.sort(sel_ref, 1) == np.sort(st["selected_experts"], 1)).all(1)
    flipped = 1.0 - same.mean()
    e_out = rel_err(out[same], r["out"][same])
    e_x1 = rel_err(st["x1"], r["x1"])
    say("block errors", dict(attn=f"{e_att:.2e}", moe_on_gpu_input=f"{e_moe:.2e}",
                             x1=f"{e_x1:.2e}", out_same_routing=f"{e_out:.2e}",
                             tokens_flipped=f"{flipped:.4f}"))
    for name, e in (("attn_out", e_att), ("moe_out", e_moe), ("x1", e_x1), ("out", e_out)):
        assert e <= 2e-2, (name, e)
    assert flipped <= 0.02, flipped
    blk.engine.close()


def test_block_small(cuda, orc):
    inp = synth.make_block_inputs(batch=2, seq_len=256, name="block-2x256")
    _check_block(orc, inp)


@pytest.mark.parametrize("pos_offset", [0, 37])
def test_block_rotates_q_in_attention_bit_exact(cuda, pos_offset):
    # The block rotates k with the RoPE kernel and q inside the attention
    # kernel as it loads it: its attention output equals that of q rotated by
    # the RoPE kernel first, bit for bit (also with a position offset).
    inp = synth.make_block_inputs(batch=2, seq_len=192, name="block-2x192")
    blk = block.PrichsBlock.from_inputs(inp)
    B, S, Hq, Hkv, hd = inp.batch, inp.seq_len, inp.n_heads, inp.n_kv_heads, inp.head_dim
    say("block q rope in attention", pos_offset)
    blk.engine.forward(dev(inp.x), B, S, pos_offset=pos_offset)
    st = blk.engine.stash()
    qkv, d = st["qkv"], Hq * hd
    q = qkv[:, :d].contiguous().view(B, S, Hq, hd)
    cos, sin = synth.rope_cache(S + pos_offset, hd, inp.rope_theta)
    cos_d, sin_d = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
    ops.rope_(q, cos_d, sin_d, S + pos_offset, B, S, pos_offset=pos_offset)
    attn = ops.attention(q.view(B * S, d), qkv[:, d:d + Hkv * hd], qkv[:, d + Hkv * hd:], B, S,
                         Hq, Hkv)
    assert torch.equal(attn.view(torch.int16), st["attn"].view(torch.int16))
    # The public entry point that rotates q on load (prichs_attention_forward_
    # rope_q) on the stashed, unrotated q: the same bits again.
    attn_rq = ops.attention(qkv[:, :d], qkv[:, d:d + Hkv * hd], qkv[:, d + Hkv * hd:], B, S, Hq,
                            Hkv, rope_q=(cos_d, sin_d, pos_offset))
    assert torch.equal(attn_rq.view(torch.int16), st["attn"].view(torch.int16))
    blk.engine.close()


@pytest.mark.parametrize("k", [1, 4])
def test_block_other_top_k(cuda, orc, k):
    # The block's final residual add rides in the combine, whose top-k is a
    # compile-time constant for k = 2 and a run-time loop otherwise: out ==
    # x1 + moe_out bit for bit (f32 and bf16) and the sub-layers against the
    # oracle, at k = 1 and k = 4.
    inp = synth.make_block_inputs(batch=1, seq_len=64, k=k, name=f"block-1x64-k{k}")
    say("block top-k", k)
    _check_block(orc, inp)


def test_block_decode_sized_residual_combine(cuda, orc):
    # At 32 tokens the block's MoE takes the decode path, followed by the
    # combine with the block's final residual add: out == x1 + moe_out bit
    # for bit (f32 and bf16), routing bit-exact and moe_out within the bf16
    # bar of the oracle on the GPU's own MoE input.
    inp = synth.make_block_inputs(batch=1, seq_len=32, name="block-1x32")
    say("block decode-sized", inp.batch, inp.seq_len)
    blk = block.PrichsBlock.from_inputs(inp)
    x = dev(inp.x)
    out = host(blk.engine.forward(x, inp.batch, inp.seq_len, out_dtype=torch.float32))
    st = {n: host(t) if t.dtype != torch.int32 else t.cpu().numpy()
          for n, t in blk.engine.stash().items()}
    np.testing.assert_array_equal(out, st["x1"] + st["moe_out"])
    out_bf = host(blk.engine.forward(x, inp.batch, inp.seq_len, out_dtype=torch.bfloat16))
    np.testing.assert_array_equal(out_bf, synth.round_bf16(st["x1"] + st["moe_out"]))
    m = inp.moe
    sub = synth.MoEInputs(**{**m.__dict__, "x": st["normed2"], "T": st["normed2"].shape[0]})
    rm = orc.moe_forward(sub)
    np.testing.assert_array_equal(st["selected_experts"], rm["sel"])
    e_row, worst = row_rel_err(st["moe_out"], rm["out"])
    assert e_row <= 2e-2, (worst, e_row)
    blk.engine.close()


def test_block_config5_full(cuda, orc):
    inp = synth.make_block_inputs()  # config 5: 4 x 2048, theta 500000
    say("block config5", inp.batch, inp.seq_len)
    _check_block(orc, inp)


def test_block_host_api_and_errors(cuda, orc):
    inp = synth.make_block_inputs(batch=1, seq_len=64, name="block-1x64")
    blk = block.PrichsBlock.from_inputs(inp)
    out = blk.forward(inp.x)  # host in, host f32 out
    dev_out = host(blk.engine.forward(dev(inp.x), 1, 64, out_dtype=torch.float32))
    np.testing.assert_array_equal(out, dev_out)  # same engine, deterministic
    from prichs_amd import _lib as L

    with pytest.raises(L.PrichsError) as e:  # more rows than the engine holds
        blk.engine.forward(dev(np.zeros((128, inp.d))), 1, 128)
    assert e.value.status == L.PRICHS_ERR_CAPACITY
    blk.engine.close()
