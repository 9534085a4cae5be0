"""Stage-level wrappers over the C ABI, on torch device tensors.

torch provides device memory and the current stream only; every computation
runs in libprichs_hip.so.  Each wrapper names the C entry point it calls.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import _lib as L

_TORCH_DTYPES = {torch.float32: L.DTYPE_F32, torch.bfloat16: L.DTYPE_BF16}
_DTYPE_TORCH = {L.DTYPE_F32: torch.float32, L.DTYPE_BF16: torch.bfloat16}


def dtype_code(t_or_dtype) -> int:
    dt = t_or_dtype.dtype if isinstance(t_or_dtype, torch.Tensor) else t_or_dtype
    if isinstance(dt, str):
        return {"f32": L.DTYPE_F32, "bf16": L.DTYPE_BF16}[dt]
    if isinstance(dt, int):
        return dt
    try:
        return _TORCH_DTYPES[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt}") from None


def torch_dtype(code: int) -> torch.dtype:
    return _DTYPE_TORCH[code]


def _p(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream(stream=None):
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


def _dev(t: torch.Tensor) -> torch.Tensor:
    if not t.is_cuda or not t.is_contiguous():
        raise ValueError("expected a contiguous device tensor")
    return t


# ------------------------------------------------------------------ router --
def router_num_blocks(T: int, E: int) -> int:
    return L.load().prichs_router_num_blocks(T, E)


def router_topk(x, w_router, router_bias, k, concept_bias=None, stream=None):
    """prichs_router_topk -> (logits f32 [T,E], idx i32 [T,k], w f32 [T,k], block_counts)."""
    lib = L.load()
    x = _dev(x)
    T, d = x.shape
    E = w_router.shape[1]
    dev = x.device
    nb = lib.prichs_router_num_blocks(T, E)
    logits = torch.empty((T, E), dtype=torch.float32, device=dev)
    idx = torch.empty((T, k), dtype=torch.int32, device=dev)
    w = torch.empty((T, k), dtype=torch.float32, device=dev)
    bc = torch.empty((max(nb * E, 1),), dtype=torch.int32, device=dev)
    nc = 0 if concept_bias is None else concept_bias.numel()
    L.check(lib.prichs_router_topk(_p(x), dtype_code(x), _p(_dev(w_router)), _p(_dev(router_bias)),
                                   _p(concept_bias), nc, T, d, E, k, _p(logits), _p(idx), _p(w),
                                   _p(bc), _stream(stream)))
    return logits, idx, w, bc


def permute(idx, w, block_counts, E, stream=None):
    """prichs_permute -> (offsets [E+2], row_token [T*k+T], row_weight [T*k], token_row [T*k])."""
    lib = L.load()
    T, k = idx.shape
    dev = idx.device
    offsets = torch.empty((E + 2,), dtype=torch.int32, device=dev)
    row_token = torch.empty((T * k + T,), dtype=torch.int32, device=dev)
    row_weight = torch.empty((T * k,), dtype=torch.float32, device=dev)
    token_row = torch.empty((T * k,), dtype=torch.int32, device=dev)
    L.check(lib.prichs_permute(_p(idx), _p(w), _p(block_counts), T, E, k, _p(offsets),
                               _p(row_token), _p(row_weight), _p(token_row), _stream(stream)))
    return offsets, row_token, row_weight, token_row


# ----------------------------------------------------------------- packing --
def _np_dtype(code):
    return np.uint16 if code == L.DTYPE_BF16 else np.float32


def pack_gate_up(gate: np.ndarray, up: np.ndarray, dtype) -> np.ndarray:
    """prichs_pack_gate_up (host): packed [Np, d] (bf16 bits as uint16, or f32;
    bf16 is fragment-tiled, see packed_rows)."""
    lib = L.load()
    code = dtype_code(dtype)
    d, f = gate.shape
    n = lib.prichs_packed_gate_up_elems(d, f, code)
    out = np.empty(n, dtype=_np_dtype(code))
    g = np.ascontiguousarray(gate, dtype=np.float32)
    u = np.ascontiguousarray(up, dtype=np.float32)
    L.check(lib.prichs_pack_gate_up(g.ctypes.data, u.ctypes.data, d, f, code, out.ctypes.data))
    return out.reshape(-1, d)


def pack_down(down: np.ndarray, dtype) -> np.ndarray:
    """prichs_pack_down (host): packed [roundup(d, 256), f] (bf16 fragment-tiled,
    see packed_rows)."""
    lib = L.load()
    code = dtype_code(dtype)
    f, d = down.shape
    n = lib.prichs_packed_down_elems(d, f, code)
    out = np.empty(n, dtype=_np_dtype(code))
    w = np.ascontiguousarray(down, dtype=np.float32)
    L.check(lib.prichs_pack_down(w.ctypes.data, d, f, code, out.ctypes.data))
    return out.reshape(-1, f)


def packed_rows(packed: np.ndarray, dtype) -> np.ndarray:
    """Logical [Np, K] rows of a packed weight.  f32 packing is row-major; bf16
    packing is fragment-major: fragment (n // 16, k // 32) is 512 contiguous
    elements, lane n % 16 + 16 * ((k % 32) // 8) holding k % 8 in 8 of them."""
    np_, K = packed.shape
    if dtype_code(dtype) != L.DTYPE_BF16:
        return packed
    t = packed.reshape(np_ // 16, K // 32, 4, 16, 8)      # [nb][ks][kq][nr][e]
    return t.transpose(0, 3, 1, 2, 4).reshape(np_, K)      # [nb][nr][ks][kq][e]


def to_device_packed(packed: list, dtype, device="cuda") -> torch.Tensor:
    """Concatenates per-expert packed arrays into one device tensor of the GEMM dtype."""
    code = dtype_code(dtype)
    host = np.concatenate([p.reshape(-1) for p in packed])
    t = torch.from_numpy(host.view(np.int16) if code == L.DTYPE_BF16 else host)
    t = t.to(device)
    return t.view(torch.bfloat16) if code == L.DTYPE_BF16 else t


# ------------------------------------------------------------------- GEMMs --
def grouped_gate_up_swiglu(x, row_token, offsets, G, rows, w_packed, d, f, stream=None,
                           out=None):
    """prichs_grouped_gate_up_swiglu -> act [rows, f] (rows = offsets[G]); out: a
    contiguous [rows, f] tensor to write (any element alignment)."""
    lib = L.load()
    act = torch.empty((rows, f), dtype=x.dtype, device=x.device) if out is None else _dev(out)
    L.check(lib.prichs_grouped_gate_up_swiglu(_p(_dev(x)), _p(row_token), _p(offsets), G, rows,
                                              _p(w_packed), d, f, dtype_code(x), _p(act),
                                              _stream(stream)))
    return act


def grouped_down(act, offsets, G, rows, w_packed, d, f, stream=None):
    """prichs_grouped_down -> y [rows, d]."""
    lib = L.load()
    y = torch.empty((rows, d), dtype=act.dtype, device=act.device)
    L.check(lib.prichs_grouped_down(_p(_dev(act)), _p(offsets), G, rows, _p(w_packed), d, f,
                                    dtype_code(act), _p(y), _stream(stream)))
    return y


def moe_combine(y, idx, w, token_row, has_shared=True, out_dtype=torch.float32, stream=None):
    """prichs_moe_combine -> out [T, d]."""
    lib = L.load()
    T, k = idx.shape
    d = y.shape[1]
    out = torch.empty((T, d), dtype=out_dtype, device=y.device)
    L.check(lib.prichs_moe_combine(_p(_dev(y)), dtype_code(y), _p(idx), _p(w), _p(token_row), T,
                                   d, k, 1 if has_shared else 0, _p(out), dtype_code(out),
                                   _stream(stream)))
    return out


# ------------------------------------------------------- memory-bound ops --
def rmsnorm(x, w, eps=1e-5, out_dtype=None, want_rstd=True, stream=None, out=None):
    """prichs_rmsnorm_forward -> (out, rstd)."""
    lib = L.load()
    x = _dev(x)
    d = x.shape[-1]
    T = x.numel() // d
    if out is None:
        out = torch.empty(x.shape, dtype=out_dtype or x.dtype, device=x.device)
    rstd = torch.empty((T,), dtype=torch.float32, device=x.device) if want_rstd else None
    L.check(lib.prichs_rmsnorm_forward(_p(x), dtype_code(x), _p(_dev(w)), _p(out), dtype_code(out),
                                       _p(rstd), T, d, eps, _stream(stream)))
    return out, rstd


def rope_(qk, cos, sin, cache_rows, batch, seq_len, pos_offset=0, sign=1, stream=None):
    """prichs_rope_forward, in place on qk [batch, seq_len, heads, head_dim]."""
    lib = L.load()
    qk = _dev(qk)
    hd = qk.shape[-1]
    H = qk.shape[-2]
    L.check(lib.prichs_rope_forward(_p(qk), dtype_code(qk), _p(_dev(cos)), _p(_dev(sin)),
                                    cache_rows, batch, seq_len, H, hd, pos_offset, sign,
                                    _stream(stream)))
    return qk


def hbm_copy(src, dst, stream=None):
    """prichs_hbm_copy: dst = src (device tensors of equal byte size, a multiple
    of 16), the library's streaming copy kernel."""
    nbytes = src.numel() * src.element_size()
    if dst.numel() * dst.element_size() != nbytes:
        raise ValueError("hbm_copy: src and dst sizes differ")
    L.check(L.load().prichs_hbm_copy(_p(src), _p(dst), nbytes, _stream(stream)))
    return dst


# ------------------------------------------------------- block sub-layers --
def pack_weight(w: np.ndarray, dtype) -> np.ndarray:
    """prichs_pack_weight (host): W [K, N] -> packed [roundup(N, 256), K]."""
    lib = L.load()
    code = dtype_code(dtype)
    K, N = w.shape
    n = lib.prichs_packed_weight_elems(K, N, code)
    out = np.empty(n, dtype=_np_dtype(code))
    wc = np.ascontiguousarray(w, dtype=np.float32)
    L.check(lib.prichs_pack_weight(wc.ctypes.data, K, N, code, out.ctypes.data))
    return out.reshape(-1, K)


def gemm(a, w_packed, N, out=None, stream=None):
    """prichs_gemm: C[M, N] = A[M, K] @ W (W packed by pack_weight / to_device_packed)."""
    lib = L.load()
    a = _dev(a)
    M, K = a.shape
    if out is None:
        out = torch.empty((M, N), dtype=a.dtype, device=a.device)
    L.check(lib.prichs_gemm(_p(a), K, M, K, _p(w_packed), N, _p(out), out.stride(0),
                            dtype_code(a), _stream(stream)))
    return out


def matmul_f32(op, a, b, out=None, stream=None):
    """prichs_matmul_f32 on f32 device tensors, in the reference's (m, k, n)
    naming: op MATMUL_AB: a [m, k] @ b [k, n]; MATMUL_ATB: a [m, k]^T @ b [m, n];
    MATMUL_ABT: a [m, k] @ b [n, k]^T.  Any sizes."""
    lib = L.load()
    a, b = _dev(a), _dev(b)
    if a.dtype != torch.float32 or b.dtype != torch.float32:
        raise TypeError("matmul_f32 takes float32 tensors")
    m, k = a.shape
    if op == L.MATMUL_AB:
        assert b.shape[0] == k
        n, shape = b.shape[1], (m, b.shape[1])
    elif op == L.MATMUL_ATB:
        assert b.shape[0] == m
        n, shape = b.shape[1], (k, b.shape[1])
    else:
        assert b.shape[1] == k
        n, shape = b.shape[0], (m, b.shape[0])
    if out is None:
        out = torch.empty(shape, dtype=torch.float32, device=a.device)
    L.check(lib.prichs_matmul_f32(op, _p(a), _p(b), _p(_dev(out)), m, k, n, _stream(stream)))
    return out


def add(a, b, out_dtype=None, stream=None):
    """prichs_add: a + b in f32 arithmetic."""
    lib = L.load()
    a, b = _dev(a), _dev(b)
    out = torch.empty(a.shape, dtype=out_dtype or a.dtype, device=a.device)
    L.check(lib.prichs_add(_p(a), dtype_code(a), _p(b), dtype_code(b), _p(out), dtype_code(out),
                           a.numel(), _stream(stream)))
    return out


def attention(q, k, v, batch, seq_len, n_heads, n_kv_heads, head_dim=128, out=None,
              stream=None, rope_q=None):
    """prichs_attention_forward on 2-D row views (rows = batch * seq_len; q/k/v may
    be column slices of one fused buffer: their row strides are passed).

    rope_q = (cos, sin, pos_offset): prichs_attention_forward_rope_q instead --
    q is rotated by RoPE as the kernel loads it (cos / sin: device f32 tables
    [cache_rows, head_dim / 2]); k must be rotated already."""
    lib = L.load()
    if out is None:
        out = torch.empty((batch * seq_len, n_heads * head_dim), dtype=q.dtype, device=q.device)
    for t in (q, k, v, out):
        if t.stride(1) != 1:
            raise ValueError("attention operands need unit column stride")
    args = (_p(q), q.stride(0), _p(k), k.stride(0), _p(v), v.stride(0), _p(out), out.stride(0),
            batch, seq_len, n_heads, n_kv_heads, head_dim, dtype_code(q))
    if rope_q is None:
        L.check(lib.prichs_attention_forward(*args, _stream(stream)))
    else:
        cos, sin, pos_offset = rope_q
        for t in (cos, sin):
            if t.dtype != torch.float32 or not t.is_contiguous() or not t.is_cuda:
                raise ValueError("rope tables must be contiguous f32 device tensors")
        cache_rows = cos.numel() // (head_dim // 2)
        L.check(lib.prichs_attention_forward_rope_q(*args, _p(cos), _p(sin), cache_rows,
                                                    pos_offset, _stream(stream)))
    return out
