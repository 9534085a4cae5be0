"""ctypes binding of libprichs_hip.so (declarations mirror include/prichs_hip.h).

The library is loaded from this package directory only; if it is missing the
import fails loudly -- there is no CPU fallback for any entry point.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# PRICHS_HIP_LIB selects another build of the same library (the sanitizer
# tests load prichs_amd/_build_asan/libprichs_hip.so this way).
LIB_PATH = os.environ.get("PRICHS_HIP_LIB") or os.path.join(HERE, "libprichs_hip.so")

PRICHS_OK = 0
PRICHS_ERR_INVALID_ARGUMENT = -1
PRICHS_ERR_CAPACITY = -2
PRICHS_ERR_HIP = -3
PRICHS_ERR_UNSUPPORTED = -4
PRICHS_ERR_STATE = -5
STATUS_NAMES = {
    0: "PRICHS_OK", -1: "PRICHS_ERR_INVALID_ARGUMENT", -2: "PRICHS_ERR_CAPACITY",
    -3: "PRICHS_ERR_HIP", -4: "PRICHS_ERR_UNSUPPORTED", -5: "PRICHS_ERR_STATE",
}
DTYPE_F32 = 0
DTYPE_BF16 = 1
MAX_EXPERTS = 64
MAX_TOPK = 8
NUM_STAGES = 6
NUM_BWD_STAGES = 10
BWD_STAGE_NAMES = ["gate_up", "rows", "dw_down", "d_act", "swiglu_bwd", "d_x_gemm", "combine",
                   "dw_gate_up", "dw_router", "total"]
STAGE_NAMES = ("router", "permute", "gate_up", "down", "combine", "total")


class PrichsError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status
        self.message = message


class MoEGrads(C.Structure):
    """prichs_moe_grads: device f32 gradient buffers (reference layouts)."""

    _fields_ = [
        ("d_router", C.c_void_p),
        ("d_gate", C.c_void_p),
        ("d_up", C.c_void_p),
        ("d_down", C.c_void_p),
        ("slot_stride", C.c_size_t),
        ("beta", C.c_int),
    ]


class MoEStash(C.Structure):
    _fields_ = [
        ("T", C.c_size_t),
        ("router_logits", C.c_void_p),
        ("selected_experts", C.c_void_p),
        ("gating_weights", C.c_void_p),
        ("offsets", C.c_void_p),
        ("row_token", C.c_void_p),
        ("row_weight", C.c_void_p),
        ("token_row", C.c_void_p),
        ("act", C.c_void_p),
        ("y", C.c_void_p),
    ]


class BlockStash(C.Structure):
    _fields_ = [
        ("T", C.c_size_t),
        ("normed1", C.c_void_p),
        ("qkv", C.c_void_p),
        ("attn", C.c_void_p),
        ("attn_out", C.c_void_p),
        ("x1", C.c_void_p),
        ("normed2", C.c_void_p),
        ("moe_out", C.c_void_p),
        ("moe", C.c_void_p),
    ]


_sz, _i, _f, _vp = C.c_size_t, C.c_int, C.c_float, C.c_void_p

# name -> (restype, argtypes)
SIGNATURES = {
    "prichs_last_error": (C.c_char_p, []),
    "prichs_clear_error": (None, []),
    "prichs_abi_version": (_i, []),
    "prichs_device_caps": (_i, [C.POINTER(_i), C.POINTER(_i), C.POINTER(_i), C.POINTER(_i)]),
    "launch_rmsnorm_forward": (None, [_vp, _vp, _vp, _vp, _sz, _sz, _f, _vp]),
    "launch_swiglu_forward": (None, [_vp, _vp, _vp, _sz, _vp]),
    "launch_rope": (None, [_vp, _vp, _vp, _sz, _sz, _sz, _i, _vp]),
    "launch_moe_gather": (None, [_vp, _vp, _vp, _sz, _sz, _vp]),
    "launch_moe_scatter_add": (None, [_vp, _vp, _vp, _vp, _sz, _sz, _vp]),
    "launch_swiglu_backward": (None, [_vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "launch_moe_backward_gather_weighted": (None, [_vp, _vp, _vp, _vp, _sz, _sz, _vp]),
    "launch_moe_router_dot": (None, [_vp, _vp, _vp, _vp, _sz, _sz, _vp]),
    "launch_moe_scatter_add_grad": (None, [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _vp]),
    "prichs_router_num_blocks": (_sz, [_sz, _sz]),
    "prichs_router_topk": (_i, [_vp, _i, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz,
                               _vp, _vp, _vp, _vp, _vp]),
    "prichs_permute": (_i, [_vp, _vp, _vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp]),
    "prichs_gate_up_interleave": (_sz, [_i]),
    "prichs_packed_gate_up_elems": (_sz, [_sz, _sz, _i]),
    "prichs_packed_down_elems": (_sz, [_sz, _sz, _i]),
    "prichs_pack_gate_up": (_i, [_vp, _vp, _sz, _sz, _i, _vp]),
    "prichs_pack_down": (_i, [_vp, _sz, _sz, _i, _vp]),
    "prichs_grouped_gate_up_swiglu": (_i, [_vp, _vp, _vp, _sz, _sz, _vp, _sz, _sz, _i, _vp, _vp]),
    "prichs_grouped_down": (_i, [_vp, _vp, _sz, _sz, _vp, _sz, _sz, _i, _vp, _vp]),
    "prichs_moe_combine": (_i, [_vp, _i, _vp, _vp, _vp, _sz, _sz, _sz, _i, _vp, _i, _vp]),
    "prichs_rmsnorm_forward": (_i, [_vp, _i, _vp, _vp, _i, _vp, _sz, _sz, _f, _vp]),
    "prichs_rope_forward": (_i, [_vp, _i, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _i, _vp]),
    "prichs_rope_cache": (_i, [_sz, _sz, _f, _vp, _vp]),
    "prichs_rope_forward_ld": (_i, [_vp, _sz, _i, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _i, _vp]),
    "prichs_add": (_i, [_vp, _i, _vp, _i, _vp, _i, _sz, _vp]),
    "prichs_hbm_copy": (_i, [_vp, _vp, _sz, _vp]),
    "prichs_packed_weight_elems": (_sz, [_sz, _sz, _i]),
    "prichs_pack_weight": (_i, [_vp, _sz, _sz, _i, _vp]),
    "prichs_gemm": (_i, [_vp, _sz, _sz, _sz, _vp, _sz, _vp, _sz, _i, _vp]),
    "prichs_attention_forward": (_i, [_vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _sz, _sz, _sz, _sz,
                                      _sz, _i, _vp]),
    "prichs_attention_forward_rope_q": (_i, [_vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _sz, _sz, _sz,
                                             _sz, _sz, _i, _vp, _vp, _sz, _sz, _vp]),
    "prichs_attention_probs_f32": (_i, [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _vp]),
    "prichs_checkpoint_open": (_i, [C.c_char_p, C.POINTER(_vp)]),
    "prichs_checkpoint_close": (_i, [_vp]),
    "prichs_checkpoint_info": (_i, [_vp, C.POINTER(C.c_uint64), C.POINTER(_f), C.POINTER(_sz),
                                    C.POINTER(_i)]),
    "prichs_checkpoint_param_len": (_i, [_vp, _sz, C.POINTER(_sz)]),
    "prichs_checkpoint_read": (_i, [_vp, _sz, _vp, _sz]),
    "prichs_checkpoint_block_param": (_sz, [_sz, _sz, _sz]),
    "prichs_moe_engine_upload_checkpoint": (_i, [_vp, _vp, _sz, _vp]),
    "prichs_block_engine_upload_checkpoint": (_i, [_vp, _vp, _sz, _vp]),
    "prichs_block_engine_create": (_i, [_sz, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _f, _f,
                                        C.POINTER(_vp)]),
    "prichs_block_engine_destroy": (_i, [_vp]),
    "prichs_block_engine_upload": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                        _vp]),
    "prichs_block_engine_forward": (_i, [_vp, _vp, _sz, _sz, _sz, _vp, _sz, _vp, _i, _vp]),
    "prichs_block_engine_stash": (_i, [_vp, C.POINTER(BlockStash)]),
    "prichs_moe_engine_create": (_i, [_sz, _sz, _sz, _sz, _sz, _i, _sz, C.POINTER(_vp)]),
    "prichs_moe_engine_destroy": (_i, [_vp]),
    "prichs_moe_engine_upload": (_i, [_vp, _vp, _vp, _vp, _vp, _vp]),
    "prichs_moe_engine_set_router_bias": (_i, [_vp, _vp]),
    "prichs_moe_engine_update_router_bias": (_i, [_vp, _f, _vp]),
    "prichs_moe_engine_get_router_bias": (_i, [_vp, _vp]),
    "prichs_moe_engine_forward": (_i, [_vp, _vp, _sz, _vp, _sz, _vp, _i, _vp]),
    "prichs_moe_engine_stash": (_i, [_vp, C.POINTER(MoEStash)]),
    "prichs_moe_engine_set_timing": (_i, [_vp, _i]),
    "prichs_moe_engine_stage_ms": (_i, [_vp, C.POINTER(_f), C.POINTER(_i)]),
    "prichs_moe_engine_enable_backward": (_i, [_vp]),
    "prichs_moe_engine_backward_stage_ms": (_i, [_vp, C.POINTER(_f), C.POINTER(_i)]),
    "prichs_moe_engine_backward": (_i, [_vp, _vp, _vp, _sz, _vp, _i, C.POINTER(MoEGrads), _i, _vp]),
    "prichs_matmul_f32": (_i, [_i, _vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    "prichs_gpu_workspace_create": (_i, [_sz, _sz, _sz, C.POINTER(_vp)]),
    "prichs_gpu_workspace_destroy": (_i, [_vp]),
    "prichs_gpu_workspace_slabs": (_i, [_vp, C.POINTER(_sz), C.POINTER(_sz), C.POINTER(_sz)]),
    "prichs_gpu_workspace_matmul": (_i, [_vp, _vp, _vp, _vp, _sz, _sz, _sz]),
    "prichs_gpu_workspace_matmul_at_b": (_i, [_vp, _vp, _vp, _vp, _sz, _sz, _sz]),
    "prichs_gpu_workspace_matmul_a_bt": (_i, [_vp, _vp, _vp, _vp, _sz, _sz, _sz]),
    "prichs_get_gpu_workspace": (_vp, []),
    "prichs_matmul_gpu": (_i, [_vp, _vp, _vp, _sz, _sz, _sz]),
    "prichs_matmul_at_b_gpu": (_i, [_vp, _vp, _vp, _sz, _sz, _sz]),
    "prichs_matmul_a_bt_gpu": (_i, [_vp, _vp, _vp, _sz, _sz, _sz]),
    "prichs_moe_forward_noalloc": (_i, [_vp, _sz, _sz, _sz, _sz, _sz, _sz, _i, _vp, _vp, _vp, _vp,
                                        _vp, _sz, _vp, _i, _vp]),
}
NOALLOC_SCRATCH_BYTES = 32 << 20
MATMUL_AB = 0
MATMUL_ATB = 1
MATMUL_ABT = 2

_lib = None


def load() -> C.CDLL:
    """Loads the in-tree libprichs_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build the HIP library first "
                "(python -c 'import __graft_entry__ as g; g.build()')")
        lib = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def last_error() -> str:
    return load().prichs_last_error().decode(errors="replace")


def check(status: int) -> None:
    if status != PRICHS_OK:
        raise PrichsError(status, last_error())
