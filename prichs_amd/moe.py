"""Host-side mirror of the reference's MoE layer interface over the C ABI.

``Expert`` / ``MoELayer`` keep the names, fields and call signatures of
crates/prichs-model/src/moe.rs:6-245 (``forward``, ``forward_with_memory``,
``forward_train`` -> (out, stash), ``update_aux_free_bias``), so tests read
like the reference's own.  The computation runs in libprichs_hip.so through a
``MoEEngine`` (the C engine handle, prichs_moe_engine_*): weights are packed
and uploaded once, and a forward is one call on a HIP stream.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib as L
from . import ops


class _DeviceView:
    """Zero-copy view of library-owned device memory for torch.as_tensor."""

    _TYPESTR = {torch.float32: "<f4", torch.int32: "<i4", torch.bfloat16: "<u2"}

    def __init__(self, ptr: int, shape, dtype: torch.dtype):
        self.__cuda_array_interface__ = {
            "shape": tuple(int(s) for s in shape),
            "typestr": self._TYPESTR[dtype],
            "data": (int(ptr), False),
            "version": 2,
            "strides": None,
        }
        self.dtype = dtype


def _device_tensor(ptr: int, shape, dtype: torch.dtype) -> torch.Tensor:
    if int(np.prod(shape)) == 0:
        return torch.empty(shape, dtype=dtype, device="cuda")
    t = torch.as_tensor(_DeviceView(ptr, shape, dtype), device="cuda")
    if dtype == torch.bfloat16:
        t = t.view(torch.bfloat16)
    return t


class MoEEngine:
    """Owner of one prichs_moe_engine handle (weights + workspace on device)."""

    def __init__(self, d: int, f: int, E: int, k: int, n_shared: int = 1, dtype="bf16",
                 max_tokens: int = 8192):
        self.lib = L.load()
        self.d, self.f, self.E, self.k, self.S = d, f, E, k, n_shared
        self.dtype = ops.dtype_code(dtype)
        self.max_tokens = max_tokens
        h = C.c_void_p()
        L.check(self.lib.prichs_moe_engine_create(d, f, E, k, n_shared, self.dtype, max_tokens,
                                                  C.byref(h)))
        self.handle = h

    def close(self):
        if getattr(self, "handle", None):
            L.check(self.lib.prichs_moe_engine_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def upload(self, w_router, router_bias, gate, up, down):
        """Reference layouts, host f32; expert lists hold the shared expert first."""
        keep = [np.ascontiguousarray(a, dtype=np.float32) for a in (*gate, *up, *down)]
        G = self.E + self.S
        arr = C.c_void_p * G
        pg = arr(*[a.ctypes.data for a in keep[:G]])
        pu = arr(*[a.ctypes.data for a in keep[G:2 * G]])
        pd = arr(*[a.ctypes.data for a in keep[2 * G:]])
        wr = np.ascontiguousarray(w_router, dtype=np.float32)
        b = None if router_bias is None else np.ascontiguousarray(router_bias, dtype=np.float32)
        L.check(self.lib.prichs_moe_engine_upload(self.handle, wr.ctypes.data,
                                                  None if b is None else b.ctypes.data,
                                                  C.cast(pg, C.c_void_p), C.cast(pu, C.c_void_p),
                                                  C.cast(pd, C.c_void_p)))

    def upload_checkpoint(self, ckpt, layer: int, router_bias=None):
        """prichs_moe_engine_upload_checkpoint: the MoE of block `layer` of an
        open ``checkpoint.Checkpoint`` (the router bias is not in the file)."""
        b = None if router_bias is None else np.ascontiguousarray(router_bias, dtype=np.float32)
        L.check(self.lib.prichs_moe_engine_upload_checkpoint(
            self.handle, ckpt.handle, layer, None if b is None else b.ctypes.data))

    def set_router_bias(self, bias):
        b = np.ascontiguousarray(bias, dtype=np.float32)
        L.check(self.lib.prichs_moe_engine_set_router_bias(self.handle, b.ctypes.data))

    def update_router_bias(self, gamma: float, stream=None):
        """prichs_moe_engine_update_router_bias: the aux-loss-free update
        (moe.rs:228-245) from the last forward's routing, on device."""
        L.check(self.lib.prichs_moe_engine_update_router_bias(self.handle, C.c_float(gamma),
                                                              ops._stream(stream)))

    def router_bias(self) -> np.ndarray:
        out = np.empty(self.E, dtype=np.float32)
        L.check(self.lib.prichs_moe_engine_get_router_bias(self.handle, out.ctypes.data))
        return out

    def forward(self, x: torch.Tensor, concept_bias: torch.Tensor | None = None,
                out: torch.Tensor | None = None, out_dtype=None, stream=None) -> torch.Tensor:
        if ops.dtype_code(x) != self.dtype:
            raise TypeError("x dtype does not match the engine dtype")
        T = x.shape[0]
        if out is None:
            od = out_dtype if out_dtype is not None else x.dtype
            out = torch.empty((T, self.d), dtype=od, device=x.device)
        nc = 0 if concept_bias is None else concept_bias.numel()
        L.check(self.lib.prichs_moe_engine_forward(
            self.handle, ops._p(ops._dev(x)), T, ops._p(concept_bias), nc, ops._p(out),
            ops.dtype_code(out), ops._stream(stream)))
        return out

    def enable_backward(self):
        """prichs_moe_engine_enable_backward: before upload."""
        L.check(self.lib.prichs_moe_engine_enable_backward(self.handle))

    def backward(self, x: torch.Tensor, d_out: torch.Tensor, grads: dict,
                 dx_weighting: int = 2, d_x: torch.Tensor | None = None, d_x_dtype=None,
                 stream=None, beta: int = 1) -> torch.Tensor:
        """prichs_moe_engine_backward after the forward of the same x.

        grads: device f32 tensors updated in place -- "d_router" [d, E] and
        "d_gate", "d_up" [G, d, f], "d_down" [G, f, d] (G = 1 + E, the shared
        expert first), or a "flat" [G, 3, d*f] buffer in the reference's
        parameter order (gate, up, down of each slot).  beta = 1 adds the
        gradients to them, beta = 0 overwrites them.  Returns d_x [T, d]."""
        for t in (x, d_out):
            if ops.dtype_code(t) != self.dtype:
                raise TypeError("x and d_out must have the engine dtype")
        T = x.shape[0]
        if d_x is None:
            od = d_x_dtype if d_x_dtype is not None else x.dtype
            d_x = torch.empty((T, self.d), dtype=od, device=x.device)
        def ptr(t):
            if t.dtype != torch.float32 or not t.is_cuda or not t.is_contiguous():
                raise ValueError("gradients are contiguous f32 device tensors")
            return t.data_ptr()

        g = L.MoEGrads()
        g.d_router = ptr(grads["d_router"])
        df = self.d * self.f
        if "flat" in grads:
            base = ptr(grads["flat"])
            g.d_gate, g.d_up, g.d_down = base, base + 4 * df, base + 8 * df
            g.slot_stride = 3 * df
        else:
            g.d_gate, g.d_up, g.d_down = (ptr(grads[k]) for k in ("d_gate", "d_up", "d_down"))
            g.slot_stride = df
        g.beta = int(beta)
        L.check(self.lib.prichs_moe_engine_backward(
            self.handle, ops._p(ops._dev(x)), ops._p(ops._dev(d_out)), T, ops._p(d_x),
            ops.dtype_code(d_x), C.byref(g), int(dx_weighting), ops._stream(stream)))
        return d_x

    def backward_stage_ms(self) -> dict:
        """Average backward stage milliseconds over the recorded backwards (plus "n")."""
        buf = (C.c_float * L.NUM_BWD_STAGES)()
        n = C.c_int(0)
        L.check(self.lib.prichs_moe_engine_backward_stage_ms(self.handle, buf, C.byref(n)))
        out = dict(zip(L.BWD_STAGE_NAMES, list(buf)))
        out["n"] = n.value
        return out

    def set_timing(self, max_forwards: int):
        """Record stage events for the next ``max_forwards`` forwards (0 = off)."""
        L.check(self.lib.prichs_moe_engine_set_timing(self.handle, int(max_forwards)))

    def stage_ms(self) -> dict:
        """Average stage milliseconds over the recorded forwards (plus "n")."""
        buf = (C.c_float * L.NUM_STAGES)()
        n = C.c_int(0)
        L.check(self.lib.prichs_moe_engine_stage_ms(self.handle, buf, C.byref(n)))
        out = dict(zip(L.STAGE_NAMES, list(buf)))
        out["n"] = n.value
        return out

    def stash(self, names=None) -> dict:
        """Device views (cloned) of the last forward's intermediates (the MoEStash);
        `names` selects a subset."""
        st = L.MoEStash()
        L.check(self.lib.prichs_moe_engine_stash(self.handle, C.byref(st)))
        T, k, E, S = st.T, self.k, self.E, self.S
        rows = T * k + S * T
        gdt = ops.torch_dtype(self.dtype)
        v = {
            "router_logits": _device_tensor(st.router_logits, (T, E), torch.float32),
            "selected_experts": _device_tensor(st.selected_experts, (T, k), torch.int32),
            "gating_weights": _device_tensor(st.gating_weights, (T, k), torch.float32),
            "offsets": _device_tensor(st.offsets, (E + 2,), torch.int32),
            "row_token": _device_tensor(st.row_token, (T * k + T,), torch.int32),
            "row_weight": _device_tensor(st.row_weight, (T * k,), torch.float32),
            "token_row": _device_tensor(st.token_row, (T * k,), torch.int32),
            "act": _device_tensor(st.act, (rows, self.f), gdt),
            "y": _device_tensor(st.y, (rows, self.d), gdt),
        }
        return {name: t.clone() for name, t in v.items() if names is None or name in names}


@dataclass
class Expert:
    """crates/prichs-model/src/moe.rs:6-10: gate/up [d, f], down [f, d] (host f32)."""

    gate_proj: np.ndarray
    up_proj: np.ndarray
    down_proj: np.ndarray


@dataclass
class MoEStash:
    """The device path's counterpart of MoEStash (moe.rs:43-53).

    Per-expert gate/up stashes do not exist on this path (SwiGLU is fused into
    the GEMM epilogue); ``act`` and ``routed_out`` hold the SwiGLU output and
    the expert outputs of every routed row in permutation order.
    """

    router_logits: np.ndarray
    selected_experts: np.ndarray
    gating_weights: np.ndarray
    expert_offsets: np.ndarray
    row_token: np.ndarray
    row_weight: np.ndarray
    act: np.ndarray
    routed_out: np.ndarray
    shared_out: np.ndarray | None


class MoELayer:
    """crates/prichs-model/src/moe.rs:58-64 with the forward running on the GPU."""

    def __init__(self, router, router_bias, shared_expert: Expert | None, experts: list,
                 top_k: int, dtype="bf16", max_tokens: int = 8192):
        self.router = np.ascontiguousarray(router, dtype=np.float32)  # [d, E]
        self.router_bias = np.ascontiguousarray(router_bias, dtype=np.float32)  # [E]
        self.shared_expert = shared_expert
        self.experts = list(experts)
        self.top_k = int(top_k)
        d, E = self.router.shape
        f = self.experts[0].gate_proj.shape[1]
        S = 1 if shared_expert is not None else 0
        self.engine = MoEEngine(d, f, E, self.top_k, S, dtype, max_tokens)
        all_e = ([shared_expert] if shared_expert is not None else []) + self.experts
        self.engine.upload(self.router, self.router_bias, [e.gate_proj for e in all_e],
                           [e.up_proj for e in all_e], [e.down_proj for e in all_e])

    @classmethod
    def from_inputs(cls, inp, max_tokens: int | None = None) -> "MoELayer":
        """Builds the layer from prichs_amd.synth.MoEInputs (shared expert first)."""
        experts = [Expert(g, u, dn) for g, u, dn in zip(inp.gate, inp.up, inp.down)]
        shared = experts[0] if inp.n_shared == 1 else None
        routed = experts[inp.n_shared:]
        return cls(inp.w_router, inp.router_bias, shared, routed, inp.k, inp.dtype,
                   max_tokens or inp.T)

    def _to_device(self, x):
        if isinstance(x, torch.Tensor) and x.is_cuda:
            return x.contiguous(), True
        xt = torch.as_tensor(np.ascontiguousarray(x, dtype=np.float32))
        tdt = ops.torch_dtype(self.engine.dtype)
        return xt.to(device="cuda", dtype=tdt).contiguous(), False

    def forward_with_memory(self, x, starkdb_concept_bias=None):
        """moe.rs:214-221.  Host arrays in -> host f32 out; device tensors stay on device."""
        xd, on_dev = self._to_device(x)
        cb = None
        if starkdb_concept_bias is not None:
            cb = torch.as_tensor(np.ascontiguousarray(starkdb_concept_bias, dtype=np.float32))
            cb = cb.to("cuda")
        out = self.engine.forward(xd, cb, out_dtype=torch.float32)
        if on_dev:
            return out
        torch.cuda.current_stream().synchronize()
        return out.cpu().numpy()

    def forward(self, x):
        """moe.rs:223-225."""
        return self.forward_with_memory(x, None)

    def forward_train(self, x, starkdb_concept_bias=None):
        """moe.rs:93-212 -> (out, MoEStash)."""
        out = self.forward_with_memory(x, starkdb_concept_bias)
        st = self.engine.stash()
        torch.cuda.current_stream().synchronize()
        T = st["selected_experts"].shape[0]
        k, S = self.top_k, self.engine.S
        h = {n: (t.view(torch.int16) if t.dtype == torch.bfloat16 else t).cpu().numpy()
             for n, t in st.items()}
        act, y = h["act"], h["y"]
        stash = MoEStash(
            router_logits=h["router_logits"], selected_experts=h["selected_experts"],
            gating_weights=h["gating_weights"], expert_offsets=h["offsets"][: self.engine.E + 1],
            row_token=h["row_token"][: T * k], row_weight=h["row_weight"], act=act[: T * k],
            routed_out=y[: T * k], shared_out=y[T * k:] if S else None)
        return out, stash

    def update_aux_free_bias_on_device(self, gamma: float = 0.001):
        """The update of the reference's training step (model.rs:1541-1547:
        counts of the last forward's selected experts, total = its tokens,
        gamma 0.001) computed on device from the permutation's group sizes;
        the host copy of the bias follows."""
        self.engine.update_router_bias(gamma)
        torch.cuda.synchronize()
        self.router_bias = self.engine.router_bias()

    def update_aux_free_bias(self, expert_token_counts, total_tokens: int, gamma: float):
        """moe.rs:228-245 (host arithmetic in f32), then pushes the bias to the engine."""
        E = len(self.experts)
        if total_tokens == 0 or E == 0:
            return
        target = np.float32(self.top_k) / np.float32(E)
        for i in range(E):
            actual = np.float32(expert_token_counts[i]) / np.float32(total_tokens)
            diff = np.float32(target - actual)
            self.router_bias[i] = np.float32(self.router_bias[i] + np.float32(gamma) * diff)
        self.engine.set_router_bias(self.router_bias)
