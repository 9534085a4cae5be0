"""ctypes front end of the CPU oracle (oracle/prichs_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as the
checker, and by bench.py's cpu_baseline leg.  The product (prichs_amd) never
imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# ORACLE_LIB selects another build (the sanitizer tests load oracle/_asan/liboracle.so).
_LIB_PATH = os.environ.get("ORACLE_LIB") or os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile (gcc, OpenMP)."""
    if force or not os.path.exists(_LIB_PATH) or (
        os.path.getmtime(_LIB_PATH) < os.path.getmtime(os.path.join(_HERE, "prichs_oracle.c"))
    ):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "liboracle.so"],
                       check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        sz = C.c_size_t
        L.orc_matmul_2d.argtypes = [_f32p, _f32p, _f32p, sz, sz, sz]
        L.orc_matmul_2d.restype = None
        L.orc_matmul_at_b.argtypes = [_f32p, _f32p, _f32p, sz, sz, sz]
        L.orc_matmul_at_b.restype = None
        L.orc_matmul_a_bt.argtypes = [_f32p, _f32p, _f32p, sz, sz, sz]
        L.orc_matmul_a_bt.restype = None
        L.orc_rms_norm.argtypes = [_f32p, _f32p, _f32p, sz, sz, C.c_float]
        L.orc_rms_norm.restype = None
        L.orc_silu.argtypes = [C.c_float]
        L.orc_silu.restype = C.c_float
        L.orc_swiglu.argtypes = [_f32p, _f32p, _f32p, sz]
        L.orc_swiglu.restype = None
        L.orc_add_tensors.argtypes = [_f32p, _f32p, _f32p, sz]
        L.orc_add_tensors.restype = None
        L.orc_top_k_gating_unbiased.argtypes = [_f32p, _f32p, sz, sz, _i32p, _f32p]
        L.orc_top_k_gating_unbiased.restype = C.c_int
        L.orc_route.argtypes = [_f32p, _f32p, _f32p, C.c_void_p, sz, sz, sz, sz, sz,
                                _f32p, _i32p, _f32p]
        L.orc_route.restype = C.c_int
        L.orc_bin_tokens.argtypes = [_i32p, _f32p, sz, sz, sz, _i32p, _i32p, _f32p, _i32p]
        L.orc_bin_tokens.restype = None
        L.orc_moe_forward.argtypes = [_f32p, sz, sz, sz, sz, sz, sz, _f32p, _f32p, C.c_void_p, sz,
                                      C.c_void_p, C.c_void_p, C.c_void_p, _f32p,
                                      _f32p, _i32p, _f32p, _i32p, _i32p, _f32p, _i32p]
        L.orc_moe_forward.restype = C.c_int
        L.orc_moe_backward.argtypes = [_f32p, _f32p, sz, sz, sz, sz, sz, _f32p, _f32p, C.c_void_p,
                                       sz, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, _f32p,
                                       _f32p, C.c_void_p, C.c_void_p, C.c_void_p]
        L.orc_moe_backward.restype = C.c_int
        L.orc_precompute_rope_cache.argtypes = [sz, sz, C.c_float, _f32p, _f32p]
        L.orc_precompute_rope_cache.restype = None
        L.orc_rope_forward_in_place.argtypes = [_f32p, _f32p, _f32p, sz, sz, sz, sz]
        L.orc_rope_forward_in_place.restype = None
        L.orc_attention_forward.argtypes = [_f32p, sz, sz, sz, sz, sz, _f32p, _f32p, _f32p, _f32p,
                                            _f32p, _f32p, sz, _f32p, C.c_void_p]
        L.orc_attention_forward.restype = C.c_int
        L.orc_block_forward.argtypes = [_f32p, sz, sz, sz, sz, sz, sz, _f32p, _f32p, C.c_float,
                                        _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, sz, sz, sz, sz,
                                        sz, _f32p, _f32p, C.c_void_p, C.c_void_p, C.c_void_p,
                                        _f32p, C.c_void_p, C.c_void_p, C.c_void_p]
        L.orc_block_forward.restype = C.c_int
        L.orc_update_aux_free_bias.argtypes = [_f32p, C.c_void_p, sz, sz, sz, C.c_float]
        L.orc_update_aux_free_bias.restype = None
        L.orc_num_threads.restype = C.c_int
        L.orc_set_num_threads.argtypes = [C.c_int]
        L.orc_set_num_threads.restype = None
        _lib = L
    return _lib


def _c(a, dt=np.float32):
    return np.ascontiguousarray(a, dtype=dt)


def num_threads() -> int:
    return lib().orc_num_threads()


def set_num_threads(n: int) -> None:
    lib().orc_set_num_threads(int(n))


def matmul_2d(a, b):
    a, b = _c(a), _c(b)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    out = np.empty((m, n), np.float32)
    lib().orc_matmul_2d(a, b, out, m, k, n)
    return out


def matmul_at_b(a, b, dw=None):
    """ops.rs:63-83 CPU branch: dw += a^T b (dw [k, n] starts at zero when None)."""
    a, b = _c(a), _c(b)
    m, k = a.shape
    m2, n = b.shape
    assert m == m2
    out = np.zeros((k, n), np.float32) if dw is None else np.array(dw, np.float32, copy=True)
    lib().orc_matmul_at_b(a, b, out, m, k, n)
    return out


def matmul_a_bt(dy, w):
    """ops.rs:85-107 CPU branch: dx = dy w^T (w [n, k])."""
    dy, w = _c(dy), _c(w)
    m, k = dy.shape
    n, k2 = w.shape
    assert k == k2
    out = np.empty((m, n), np.float32)
    lib().orc_matmul_a_bt(dy, w, out, m, k, n)
    return out


def rms_norm(x, w, eps=1e-5):
    x, w = _c(x), _c(w)
    out = np.empty_like(x)
    d = x.shape[-1]
    lib().orc_rms_norm(x, w, out, x.size // d, d, eps)
    return out


def silu(v: float) -> float:
    return lib().orc_silu(float(v))


def swiglu(g, u):
    g, u = _c(g), _c(u)
    out = np.empty_like(g)
    lib().orc_swiglu(g, u, out, g.size)
    return out


def add_tensors(a, b):
    a, b = _c(a), _c(b)
    out = np.empty_like(a)
    lib().orc_add_tensors(a, b, out, a.size)
    return out


def top_k_gating_unbiased(raw, adj, k):
    raw, adj = _c(raw), _c(adj)
    E = raw.size
    idx = np.empty(k, np.int32)
    w = np.empty(k, np.float32)
    rc = lib().orc_top_k_gating_unbiased(raw, adj, E, k, idx, w)
    if rc != 0:
        raise ValueError("bad top-k arguments")
    return idx, w


def route(x, w_router, router_bias, k, concept_bias=None):
    x, w_router, router_bias = _c(x), _c(w_router), _c(router_bias)
    T, d = x.shape
    E = w_router.shape[1]
    logits = np.empty((T, E), np.float32)
    sel = np.empty((T, k), np.int32)
    gw = np.empty((T, k), np.float32)
    cb = None if concept_bias is None else _c(concept_bias)
    rc = lib().orc_route(x, w_router, router_bias, None if cb is None else cb.ctypes.data,
                         0 if cb is None else cb.size, T, d, E, k, logits, sel, gw)
    if rc != 0:
        raise ValueError("bad routing arguments")
    return logits, sel, gw


def bin_tokens(sel, gw, E):
    sel, gw = _c(sel, np.int32), _c(gw)
    T, k = sel.shape
    offsets = np.empty(E + 1, np.int32)
    row_token = np.empty(T * k, np.int32)
    row_weight = np.empty(T * k, np.float32)
    token_row = np.empty(T * k, np.int32)
    lib().orc_bin_tokens(sel, gw, T, E, k, offsets, row_token, row_weight, token_row)
    return offsets, row_token, row_weight, token_row


def update_aux_free_bias(bias, counts, top_k, total_tokens, gamma):
    """MoELayer::update_aux_free_bias (moe.rs:228-245) on a copy of bias."""
    b = _c(bias).copy()
    cnt = np.ascontiguousarray(counts, dtype=np.int64)
    lib().orc_update_aux_free_bias(b, cnt.ctypes.data, b.size, top_k, total_tokens,
                                   C.c_float(gamma))
    return b


def moe_forward(inp, concept_bias=None):
    """MoELayer::forward_train (moe.rs:93-212) on a synth.MoEInputs; returns a dict."""
    T, d, f, E, k, S = inp.T, inp.d, inp.f, inp.E, inp.k, inp.n_shared
    x = _c(inp.x)
    gates = [_c(a) for a in inp.gate]
    ups = [_c(a) for a in inp.up]
    downs = [_c(a) for a in inp.down]
    arr_t = C.c_void_p * (S + E)
    pg = arr_t(*[a.ctypes.data for a in gates])
    pu = arr_t(*[a.ctypes.data for a in ups])
    pd = arr_t(*[a.ctypes.data for a in downs])
    out = np.empty((T, d), np.float32)
    logits = np.empty((T, E), np.float32)
    sel = np.empty((T, k), np.int32)
    gw = np.empty((T, k), np.float32)
    offsets = np.empty(E + 1, np.int32)
    row_token = np.empty(max(T * k, 1), np.int32)
    row_weight = np.empty(max(T * k, 1), np.float32)
    token_row = np.empty(max(T * k, 1), np.int32)
    cb = None if concept_bias is None else _c(concept_bias)
    rc = lib().orc_moe_forward(x, T, d, f, E, k, S, _c(inp.w_router), _c(inp.router_bias),
                               None if cb is None else cb.ctypes.data, 0 if cb is None else cb.size,
                               C.cast(pg, C.c_void_p), C.cast(pu, C.c_void_p), C.cast(pd, C.c_void_p),
                               out, logits, sel, gw, offsets, row_token, row_weight, token_row)
    if rc != 0:
        raise RuntimeError("oracle moe_forward failed")
    return dict(out=out, logits=logits, sel=sel, gw=gw, offsets=offsets,
                row_token=row_token[: T * k], row_weight=row_weight[: T * k],
                token_row=token_row[: T * k])


def moe_backward(inp, d_out, dx_weighting=2, concept_bias=None, grads=None):
    """The MoE backward (engine.rs:2242-2789 driven as model.rs:1474-1561; router VJP
    backward.rs:269-287) on a synth.MoEInputs with n_shared = 1.  Returns
    dict(d_x, d_router, d_gate, d_up, d_down); gradients start from `grads` (a dict
    of the same keys, copied) or zeros, and are accumulated into."""
    T, d, f, E, k, S = inp.T, inp.d, inp.f, inp.E, inp.k, inp.n_shared
    if S != 1:
        raise ValueError("the reference backward has one shared expert")
    x = _c(inp.x)
    dout = _c(d_out)
    gates, ups, downs = ([_c(a) for a in inp.gate], [_c(a) for a in inp.up],
                         [_c(a) for a in inp.down])
    G = S + E
    if grads is None:
        grads = dict(d_router=np.zeros((d, E), np.float32),
                     d_gate=[np.zeros((d, f), np.float32) for _ in range(G)],
                     d_up=[np.zeros((d, f), np.float32) for _ in range(G)],
                     d_down=[np.zeros((f, d), np.float32) for _ in range(G)])
    out = dict(d_x=np.empty((T, d), np.float32), d_router=_c(grads["d_router"]).copy(),
               d_gate=[_c(a).copy() for a in grads["d_gate"]],
               d_up=[_c(a).copy() for a in grads["d_up"]],
               d_down=[_c(a).copy() for a in grads["d_down"]])
    arr = C.c_void_p * G
    ptrs = lambda lst: C.cast(arr(*[a.ctypes.data for a in lst]), C.c_void_p)  # noqa: E731
    cb = None if concept_bias is None else _c(concept_bias)
    rc = lib().orc_moe_backward(x, dout, T, d, f, E, k, _c(inp.w_router), _c(inp.router_bias),
                                None if cb is None else cb.ctypes.data,
                                0 if cb is None else cb.size, ptrs(gates), ptrs(ups), ptrs(downs),
                                dx_weighting, out["d_x"], out["d_router"], ptrs(out["d_gate"]),
                                ptrs(out["d_up"]), ptrs(out["d_down"]))
    if rc != 0:
        raise RuntimeError("oracle moe_backward failed")
    return out


def precompute_rope_cache(max_seq_len, head_dim, theta):
    half = head_dim // 2
    cos = np.empty(max_seq_len * half, np.float32)
    sin = np.empty(max_seq_len * half, np.float32)
    lib().orc_precompute_rope_cache(max_seq_len, head_dim, theta, cos, sin)
    return cos, sin


def rope_forward(t, cos, sin, pos_offset=0):
    """Returns a rotated copy of t [seq, heads, head_dim] (backward.rs:160-188)."""
    t = np.array(t, dtype=np.float32, copy=True, order="C")
    S, H, hd = t.shape
    lib().orc_rope_forward_in_place(t, _c(cos), _c(sin), S, H, hd, pos_offset)
    return t


def attention_forward(x, Hq, Hkv, wq, wk, wv, wo, cos, sin, pos_offset=0, want_concat=False):
    """SelfAttention::forward_with_rope (attention.rs:56-176) of one sequence x [S, d]."""
    x = _c(x)
    S, d = x.shape
    hd = d // Hq
    out = np.empty((S, d), np.float32)
    cat = np.empty((S, d), np.float32) if want_concat else None
    rc = lib().orc_attention_forward(x, S, d, Hq, Hkv, hd, _c(wq), _c(wk), _c(wv), _c(wo),
                                     _c(cos), _c(sin), pos_offset, out,
                                     None if cat is None else cat.ctypes.data)
    if rc != 0:
        raise ValueError("bad attention arguments")
    return (out, cat) if want_concat else out


def block_forward(inp):
    """PrichsBlock::forward_with_rope (block.rs:50-68) over inp.batch sequences
    (a prichs_amd.synth.BlockInputs); returns dict(out, attn, x1, moe)."""
    m = inp.moe
    T, d = inp.x.shape
    S, E, k, n_sh = m.n_shared + m.E, m.E, m.k, m.n_shared
    gates = [_c(a) for a in m.gate]
    ups = [_c(a) for a in m.up]
    downs = [_c(a) for a in m.down]
    arr_t = C.c_void_p * S
    pg = arr_t(*[a.ctypes.data for a in gates])
    pu = arr_t(*[a.ctypes.data for a in ups])
    pd = arr_t(*[a.ctypes.data for a in downs])
    out = np.empty((T, d), np.float32)
    attn = np.empty((T, d), np.float32)
    x1 = np.empty((T, d), np.float32)
    mo = np.empty((T, d), np.float32)
    rc = lib().orc_block_forward(
        _c(inp.x), inp.batch, inp.seq_len, d, inp.n_heads, inp.n_kv_heads, inp.head_dim,
        _c(inp.input_norm), _c(inp.post_norm), inp.eps, _c(inp.wq), _c(inp.wk), _c(inp.wv),
        _c(inp.wo), _c(inp.cos), _c(inp.sin), 0, m.f, E, k, n_sh, _c(m.w_router),
        _c(m.router_bias), C.cast(pg, C.c_void_p), C.cast(pu, C.c_void_p),
        C.cast(pd, C.c_void_p), out, attn.ctypes.data, x1.ctypes.data, mo.ctypes.data)
    if rc != 0:
        raise RuntimeError("oracle block_forward failed")
    return dict(out=out, attn=attn, x1=x1, moe=mo)
