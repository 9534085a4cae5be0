"""Host-side mirror of the reference's PrichsBlock over the C ABI.

``SelfAttention`` and ``PrichsBlock`` keep the fields and call shape of
crates/prichs-model/src/attention.rs:17-26 and crates/prichs-model/src/
block.rs:15-82 (``forward_with_rope``, ``forward``); the computation runs in
libprichs_hip.so through a ``BlockEngine`` (prichs_block_engine_*): RMSNorm,
one fused QKV GEMM, RoPE, causal GQA flash attention, the output projection,
the residual, RMSNorm, the MoE engine and the second residual.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib as L
from . import ops
from .moe import Expert, _device_tensor


class BlockEngine:
    """Owner of one prichs_block_engine handle (bf16 weights and workspace)."""

    def __init__(self, d, n_heads, n_kv_heads, f, E, k, n_shared=1, max_tokens=8192,
                 max_seq_len=2048, rope_theta=10000.0, eps=1e-5):
        self.lib = L.load()
        self.d, self.Hq, self.Hkv, self.f, self.E, self.k, self.S = (
            d, n_heads, n_kv_heads, f, E, k, n_shared)
        self.hd = d // n_heads
        self.max_tokens = max_tokens
        h = C.c_void_p()
        L.check(self.lib.prichs_block_engine_create(d, n_heads, n_kv_heads, f, E, k, n_shared,
                                                    max_tokens, max_seq_len,
                                                    C.c_float(rope_theta), C.c_float(eps),
                                                    C.byref(h)))
        self.handle = h

    def close(self):
        if getattr(self, "handle", None):
            L.check(self.lib.prichs_block_engine_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def upload(self, input_norm, post_attn_norm, wq, wk, wv, wo, w_router, router_bias, gate,
               up, down):
        f32 = lambda a: np.ascontiguousarray(a, dtype=np.float32)  # noqa: E731
        dense = [f32(a) for a in (input_norm, post_attn_norm, wq, wk, wv, wo, w_router)]
        bias = f32(router_bias)
        keep = [f32(a) for a in (*gate, *up, *down)]
        G = self.E + self.S
        arr = C.c_void_p * G
        pg = arr(*[a.ctypes.data for a in keep[:G]])
        pu = arr(*[a.ctypes.data for a in keep[G:2 * G]])
        pd = arr(*[a.ctypes.data for a in keep[2 * G:]])
        L.check(self.lib.prichs_block_engine_upload(
            self.handle, *[a.ctypes.data for a in dense[:6]], dense[6].ctypes.data,
            bias.ctypes.data, C.cast(pg, C.c_void_p), C.cast(pu, C.c_void_p),
            C.cast(pd, C.c_void_p)))

    def upload_checkpoint(self, ckpt, layer: int, router_bias=None):
        """prichs_block_engine_upload_checkpoint: norms, attention and MoE of
        block `layer` of an open ``checkpoint.Checkpoint``."""
        b = None if router_bias is None else np.ascontiguousarray(router_bias, dtype=np.float32)
        L.check(self.lib.prichs_block_engine_upload_checkpoint(
            self.handle, ckpt.handle, layer, None if b is None else b.ctypes.data))

    def forward(self, x: torch.Tensor, batch: int, seq_len: int, pos_offset: int = 0,
                concept_bias: torch.Tensor | None = None, out: torch.Tensor | None = None,
                out_dtype=None, stream=None) -> torch.Tensor:
        if x.dtype != torch.bfloat16 or not x.is_cuda or not x.is_contiguous():
            raise TypeError("x must be a contiguous bf16 device tensor")
        if out is None:
            out = torch.empty(x.shape, dtype=out_dtype or x.dtype, device=x.device)
        nc = 0 if concept_bias is None else concept_bias.numel()
        L.check(self.lib.prichs_block_engine_forward(
            self.handle, ops._p(x), batch, seq_len, pos_offset, ops._p(concept_bias), nc,
            ops._p(out), ops.dtype_code(out), ops._stream(stream)))
        return out

    def stash(self) -> dict:
        """Device copies of the last forward's intermediates."""
        st = L.BlockStash()
        L.check(self.lib.prichs_block_engine_stash(self.handle, C.byref(st)))
        T, d, n = st.T, self.d, self.d + 2 * self.Hkv * self.hd
        bf = torch.bfloat16
        v = {
            "normed1": _device_tensor(st.normed1, (T, d), bf),
            "qkv": _device_tensor(st.qkv, (T, n), bf),
            "attn": _device_tensor(st.attn, (T, d), bf),
            "attn_out": _device_tensor(st.attn_out, (T, d), bf),
            "x1": _device_tensor(st.x1, (T, d), torch.float32),
            "normed2": _device_tensor(st.normed2, (T, d), bf),
            "moe_out": _device_tensor(st.moe_out, (T, d), bf),
        }
        ms = L.MoEStash()
        L.check(self.lib.prichs_moe_engine_stash(C.c_void_p(st.moe), C.byref(ms)))
        v["selected_experts"] = _device_tensor(ms.selected_experts, (T, self.k), torch.int32)
        v["gating_weights"] = _device_tensor(ms.gating_weights, (T, self.k), torch.float32)
        v["router_logits"] = _device_tensor(ms.router_logits, (T, self.E), torch.float32)
        return {name: t.clone() for name, t in v.items()}


@dataclass
class SelfAttention:
    """crates/prichs-model/src/attention.rs:17-26 (host f32, [K, N] layouts)."""

    q_proj: np.ndarray
    k_proj: np.ndarray
    v_proj: np.ndarray
    out_proj: np.ndarray
    hidden_dim: int
    num_heads: int
    num_kv_heads: int
    head_dim: int


class PrichsBlock:
    """crates/prichs-model/src/block.rs:15-82 with the forward on the GPU.

    ``moe`` is a dict of the MoE sub-layer (router, router_bias, shared_expert,
    experts, top_k) in the reference layouts.  The RoPE tables are built by the
    engine for ``rope_theta`` (backward.rs:136-157), as forward() does with
    theta = 10000 (block.rs:70-82).
    """

    def __init__(self, input_norm, attention: SelfAttention, post_attn_norm, moe: dict,
                 eps: float = 1e-5, rope_theta: float = 10000.0, max_tokens: int = 8192,
                 max_seq_len: int = 2048):
        self.input_norm = np.ascontiguousarray(input_norm, dtype=np.float32)
        self.attention = attention
        self.post_attn_norm = np.ascontiguousarray(post_attn_norm, dtype=np.float32)
        self.moe = moe
        self.eps = float(eps)
        a = attention
        experts = ([moe["shared_expert"]] if moe.get("shared_expert") is not None else []) + \
            list(moe["experts"])
        self.engine = BlockEngine(a.hidden_dim, a.num_heads, a.num_kv_heads,
                                  moe["experts"][0].gate_proj.shape[1], len(moe["experts"]),
                                  moe["top_k"], 1 if moe.get("shared_expert") is not None else 0,
                                  max_tokens, max(max_seq_len, 1024), rope_theta, eps)
        self.engine.upload(self.input_norm, self.post_attn_norm, a.q_proj, a.k_proj, a.v_proj,
                           a.out_proj, moe["router"], moe["router_bias"],
                           [e.gate_proj for e in experts], [e.up_proj for e in experts],
                           [e.down_proj for e in experts])

    @classmethod
    def from_inputs(cls, inp, max_tokens: int | None = None) -> "PrichsBlock":
        """Builds the block from prichs_amd.synth.BlockInputs."""
        m = inp.moe
        experts = [Expert(g, u, dn) for g, u, dn in zip(m.gate, m.up, m.down)]
        moe = dict(router=m.w_router, router_bias=m.router_bias, top_k=m.k,
                   shared_expert=experts[0] if m.n_shared else None,
                   experts=experts[m.n_shared:])
        att = SelfAttention(inp.wq, inp.wk, inp.wv, inp.wo, inp.d, inp.n_heads, inp.n_kv_heads,
                            inp.head_dim)
        return cls(inp.input_norm, att, inp.post_norm, moe, inp.eps, inp.rope_theta,
                   max_tokens or inp.batch * inp.seq_len, max(inp.seq_len, 1024))

    def forward_with_rope(self, x, pos_offset: int = 0, starkdb_concept_bias=None,
                          batch: int = 1):
        """block.rs:50-68 for `batch` sequences stacked along rows.  Host arrays in
        -> host f32 out; bf16 device tensors stay on the device."""
        on_dev = isinstance(x, torch.Tensor) and x.is_cuda
        if on_dev:
            xd = x.contiguous()
        else:
            xd = torch.as_tensor(np.ascontiguousarray(x, dtype=np.float32)).to(
                device="cuda", dtype=torch.bfloat16).contiguous()
        rows = xd.shape[0]
        if rows % batch:
            raise ValueError("rows must be a multiple of batch")
        cb = None
        if starkdb_concept_bias is not None:
            cb = torch.as_tensor(np.ascontiguousarray(starkdb_concept_bias, np.float32)).to("cuda")
        out = self.engine.forward(xd, batch, rows // batch, pos_offset, cb,
                                  out_dtype=torch.float32)
        if on_dev:
            return out
        torch.cuda.current_stream().synchronize()
        return out.cpu().numpy()

    def forward(self, x, starkdb_concept_bias=None, batch: int = 1):
        """block.rs:70-82 (positions from 0)."""
        return self.forward_with_rope(x, 0, starkdb_concept_bias, batch)
