"""Reference weight files (.prichs) on the C ABI: read, index, upload.

Mirrors Model::save_checkpoint / Model::load_checkpoint
(crates/prichs-model/src/model.rs:1648-1736) and the parameter order of
Model::get_parameter_tensors (model.rs:312-338).  ``Checkpoint`` wraps
prichs_checkpoint_* (the reader lives in libprichs_hip.so, so every caller of
the C ABI reads files the same way); ``write_prichs02`` writes the PRICHS02
layout exactly as save_checkpoint does, for fixtures and for tools that
produce weights outside the reference.
"""
from __future__ import annotations

import ctypes as C
import struct

import numpy as np

from . import _lib as L

MAGIC_V2 = b"PRICHS02"
MAGIC_LEGACY = b"PRICHS_W"

# Block slots (model.rs:318-333); expert e's gate/up/down are EXPERT0 + 3e + 0/1/2.
INPUT_NORM, Q_PROJ, K_PROJ, V_PROJ, OUT_PROJ, POST_ATTN_NORM, ROUTER = range(7)
SHARED_GATE, SHARED_UP, SHARED_DOWN, EXPERT0 = 7, 8, 9, 10


def block_param(layer: int, E: int, slot: int) -> int:
    """prichs_checkpoint_block_param: index of `slot` of block `layer`."""
    idx = L.load().prichs_checkpoint_block_param(layer, E, slot)
    if idx == C.c_size_t(-1).value:
        raise IndexError(f"slot {slot} outside a block of {10 + 3 * E} parameters")
    return idx


def write_prichs02(path, step: int, loss: float, tensors) -> None:
    """save_checkpoint (model.rs:1648-1670): magic, step u64, loss f32,
    count u64, then per tensor its element count u64 and its f32 data."""
    with open(path, "wb") as fh:
        fh.write(MAGIC_V2)
        fh.write(struct.pack("<Q", step))
        fh.write(struct.pack("<f", loss))
        fh.write(struct.pack("<Q", len(tensors)))
        for t in tensors:
            a = np.ascontiguousarray(t, dtype="<f4").reshape(-1)
            fh.write(struct.pack("<Q", a.size))
            fh.write(a.tobytes())


class Checkpoint:
    """An open weight file (prichs_checkpoint handle)."""

    def __init__(self, path):
        self.lib = L.load()
        h = C.c_void_p()
        L.check(self.lib.prichs_checkpoint_open(str(path).encode(), C.byref(h)))
        self.handle = h
        step, loss = C.c_uint64(), C.c_float()
        n, fmt = C.c_size_t(), C.c_int()
        L.check(self.lib.prichs_checkpoint_info(h, C.byref(step), C.byref(loss), C.byref(n),
                                                C.byref(fmt)))
        self.step, self.loss, self.n_params, self.format = step.value, loss.value, n.value, fmt.value

    def close(self):
        if getattr(self, "handle", None):
            L.check(self.lib.prichs_checkpoint_close(self.handle))
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def param_len(self, index: int) -> int:
        n = C.c_size_t()
        L.check(self.lib.prichs_checkpoint_param_len(self.handle, index, C.byref(n)))
        return n.value

    def read(self, index: int) -> np.ndarray:
        """Parameter `index` as a flat float32 array (bit patterns kept)."""
        out = np.empty(self.param_len(index), dtype=np.float32)
        L.check(self.lib.prichs_checkpoint_read(self.handle, index, out.ctypes.data, out.size))
        return out
