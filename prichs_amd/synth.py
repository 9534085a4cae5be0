"""Seeded synthetic inputs for the PRICHS MoE configurations.

The reference draws weights with an unseeded ``rand::thread_rng()`` and a
Box-Muller transform (crates/prichs-core/src/tensor.rs:49-63), so its inputs
cannot be reproduced.  This module owns a seeded, counter-based generator with
the same transform:

* SplitMix64 (Steele, Lea, Flood 2014) over a 64-bit counter: draw ``i`` of a
  generator seeded with ``s`` is ``mix(s + (i + 1) * 0x9E3779B97F4A7C15)``.
* A uniform is the top 24 bits of a draw, mapped to (0, 1]:
  ``((z >> 40) + 1) * 2**-24`` (exact in f32).
* One normal sample takes two uniforms ``u1, u2``; like tensor.rs:57-60,
  ``u1 = max(u1, 1e-7)`` and ``z0 = sqrt(-2 ln u1) * cos(2 pi u2)``.  ``z0`` is
  evaluated in float64 and rounded once to f32; the sample is then
  ``mean + z0 * std`` in f32 arithmetic (product rounded, then sum).

Tensors are drawn in a fixed order (x, router weights, router bias, shared
expert gate/up/down, routed experts 0..E-1 gate/up/down), each consuming
``2 * numel`` draws from one running counter.  bf16 configurations round every
drawn tensor except the router bias to bf16 (round to nearest even) and hand
the rounded values, upcast to f32, to both the GPU path and the CPU oracle, so
both see identical numbers.
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass, field

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 22


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


class SplitMixNormal:
    """Counter-based SplitMix64 + Box-Muller normal generator."""

    def __init__(self, seed: int = 0):
        self.seed = np.uint64(seed & 0xFFFFFFFFFFFFFFFF)
        self.counter = 0  # number of 64-bit draws consumed so far

    def uniform(self, n: int) -> np.ndarray:
        """``n`` uniforms in (0, 1] as float32, consuming ``n`` draws."""
        out = np.empty(n, dtype=np.float32)
        with np.errstate(over="ignore"):
            for s in range(0, n, _CHUNK):
                e = min(n, s + _CHUNK)
                i = np.arange(self.counter + s + 1, self.counter + e + 1, dtype=np.uint64)
                z = _mix(self.seed + i * _GOLDEN)
                out[s:e] = ((z >> np.uint64(40)) + np.uint64(1)).astype(np.float32) * np.float32(2.0**-24)
        self.counter += n
        return out

    def randn(self, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
        shape = (shape,) if isinstance(shape, int) else tuple(shape)
        n = int(np.prod(shape))
        out = np.empty(n, dtype=np.float32)
        m32, s32 = np.float32(mean), np.float32(std)
        for s in range(0, n, _CHUNK):
            e = min(n, s + _CHUNK)
            u = self.uniform(2 * (e - s)).reshape(-1, 2)
            u1 = np.maximum(u[:, 0], np.float32(1e-7)).astype(np.float64)
            u2 = u[:, 1].astype(np.float64)
            z0 = (np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)).astype(np.float32)
            out[s:e] = m32 + z0 * s32
        return out.reshape(shape)


def round_bf16(a: np.ndarray) -> np.ndarray:
    """Round float32 values to bf16 (nearest even); returns float32 holding them."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    bits = a.view(np.uint32)
    rounded = (bits + np.uint32(0x7FFF) + ((bits >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)
    nan = np.isnan(a)
    rounded = np.where(nan, (bits | np.uint32(0x00400000)) & np.uint32(0xFFFF0000), rounded)
    return rounded.view(np.float32)


def to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) of float32 values that are already bf16-exact."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    return (a.view(np.uint32) >> np.uint32(16)).astype(np.uint16)


def from_bf16_bits(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def rms_norm_rows(x: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    """Row RMSNorm with unit weights, evaluated in float64 (input preparation only)."""
    x64 = x.astype(np.float64)
    inv = 1.0 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + eps)
    return (x64 * inv).astype(np.float32)


@dataclass
class MoEInputs:
    """One MoE layer's inputs in the reference's layouts (all float32).

    gate/up: [d, f]; down: [f, d]; router: [d, E] (crates/prichs-model/src/moe.rs:16-18, 74).
    Lists hold the shared expert first (when n_shared == 1), then routed experts 0..E-1.
    """

    name: str
    T: int
    d: int
    f: int
    E: int
    k: int
    n_shared: int
    dtype: str  # "f32" or "bf16": arithmetic type of the GPU path
    x: np.ndarray
    w_router: np.ndarray
    router_bias: np.ndarray
    gate: list = field(default_factory=list)
    up: list = field(default_factory=list)
    down: list = field(default_factory=list)
    concept_bias: np.ndarray | None = None

    def digest(self) -> str:
        h = hashlib.sha256()
        for a in [self.x, self.w_router, self.router_bias, *self.gate, *self.up, *self.down]:
            h.update(np.ascontiguousarray(a, dtype=np.float32).tobytes())
        return h.hexdigest()


# Router bias that sends about 60% of the assignments to experts 0 and 1 at
# config 3 (bias[0] = bias[1] = beta, others 0).  Found by bisection on the
# routing of the seed-0 inputs: beta = 1.0 gives 59.95% (19,646 of 32,768
# assignments; about 9.8k rows on each of experts 0/1 and 2.1-2.3k on the rest).
SKEW_BETA_CONFIG3 = 1.0

CONFIGS = {
    1: dict(T=512, d=256, f=128, E=8, k=2, n_shared=1, dtype="f32", x_norm=False, bias_std=0.0),
    2: dict(T=8192, d=1536, f=1280, E=8, k=2, n_shared=1, dtype="bf16", x_norm=True, bias_std=0.01),
    3: dict(T=16384, d=1536, f=1280, E=8, k=2, n_shared=1, dtype="bf16", x_norm=True, bias_std=None),
    4: dict(T=32, d=1536, f=1280, E=8, k=2, n_shared=1, dtype="bf16", x_norm=True, bias_std=0.01),
}


def make_moe_inputs(T: int, d: int, f: int, E: int = 8, k: int = 2, n_shared: int = 1,
                    dtype: str = "bf16", x_norm: bool = True, bias_std: float | None = 0.01,
                    skew_beta: float = SKEW_BETA_CONFIG3, w_std: float = 0.02, seed: int = 0,
                    name: str = "custom") -> MoEInputs:
    g = SplitMixNormal(seed)
    x = g.randn((T, d), 0.0, 1.0)
    if x_norm:
        x = rms_norm_rows(x)
    w_router = g.randn((d, E), 0.0, w_std)
    if bias_std is None:  # skewed configuration
        router_bias = np.zeros(E, dtype=np.float32)
        router_bias[: min(2, E)] = np.float32(skew_beta)
    elif bias_std == 0.0:
        router_bias = np.zeros(E, dtype=np.float32)
    else:
        router_bias = g.randn((E,), 0.0, bias_std)
    gate, up, down = [], [], []
    for _ in range(n_shared + E):
        gate.append(g.randn((d, f), 0.0, w_std))
        up.append(g.randn((d, f), 0.0, w_std))
        down.append(g.randn((f, d), 0.0, w_std))
    if dtype == "bf16":
        x = round_bf16(x)
        w_router = round_bf16(w_router)
        gate = [round_bf16(a) for a in gate]
        up = [round_bf16(a) for a in up]
        down = [round_bf16(a) for a in down]
    return MoEInputs(name=name, T=T, d=d, f=f, E=E, k=k, n_shared=n_shared, dtype=dtype,
                     x=x, w_router=w_router, router_bias=router_bias, gate=gate, up=up, down=down)


def config_inputs(cfg: int, seed: int = 0, **overrides) -> MoEInputs:
    """Inputs of BASELINE configuration ``cfg`` (1-4); ``overrides`` replace shape keys."""
    c = dict(CONFIGS[cfg])
    c.update(overrides)
    return make_moe_inputs(seed=seed, name=f"config{cfg}", **c)


@dataclass
class BlockInputs:
    """One PrichsBlock's inputs (crates/prichs-model/src/block.rs:15-48) for
    `batch` independent sequences of `seq_len` rows, reference layouts, f32.

    x [batch * seq_len, d]; wq/wo [d, d]; wk/wv [d, n_kv_heads * head_dim];
    input_norm/post_norm [d]; cos/sin the RoPE cache [cache_rows, head_dim/2]
    (crates/prichs-core/src/backward.rs:136-157) for rope_theta; moe the
    MoE sub-layer's MoEInputs (its x is unused).
    """

    name: str
    batch: int
    seq_len: int
    d: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    rope_theta: float
    eps: float
    dtype: str
    x: np.ndarray
    input_norm: np.ndarray
    post_norm: np.ndarray
    wq: np.ndarray
    wk: np.ndarray
    wv: np.ndarray
    wo: np.ndarray
    cos: np.ndarray
    sin: np.ndarray
    moe: MoEInputs

    def digest(self) -> str:
        """SHA-256 of every input tensor as little-endian f32 bytes, in a fixed
        order: x, the norms, the projections, then the MoE's router, bias and
        expert weights (shared first)."""
        h = hashlib.sha256()
        m = self.moe
        for a in [self.x, self.input_norm, self.post_norm, self.wq, self.wk, self.wv, self.wo,
                  m.w_router, m.router_bias, *m.gate, *m.up, *m.down]:
            h.update(np.ascontiguousarray(a, dtype=np.float32).tobytes())
        return h.hexdigest()


def rope_cache(max_seq_len: int, head_dim: int, theta: float):
    """(cos, sin) RoPE tables [max_seq_len * head_dim/2] from the library's host
    function prichs_rope_cache (backward.rs:136-157 with libm)."""
    import ctypes as C

    from . import _lib

    half = head_dim // 2
    cos = np.empty(max_seq_len * half, np.float32)
    sin = np.empty(max_seq_len * half, np.float32)
    _lib.check(_lib.load().prichs_rope_cache(max_seq_len, head_dim, C.c_float(theta),
                                             cos.ctypes.data, sin.ctypes.data))
    return cos, sin


def make_block_inputs(batch: int = 4, seq_len: int = 2048, d: int = 1536, n_heads: int = 12,
                      n_kv_heads: int = 3, f: int = 1280, E: int = 8, k: int = 2,
                      n_shared: int = 1, rope_theta: float = 500000.0, dtype: str = "bf16",
                      w_std: float = 0.02, seed: int = 0, name: str = "config5",
                      cos_sin=None) -> BlockInputs:
    """Configuration 5 by default: 4 x 2048 rows of x ~ N(0,1), every weight
    ~ N(0, 0.02), norm weights ~ N(1, 0.02) (block.rs:25-26), router bias 0
    (moe.rs:75), RoPE theta 500000; bf16 rounds every drawn tensor.
    cos_sin may supply the RoPE cache (e.g. the oracle's glibc table)."""
    g = SplitMixNormal(seed)
    hd = d // n_heads
    T = batch * seq_len
    x = g.randn((T, d), 0.0, 1.0)
    input_norm = g.randn((d,), 1.0, w_std)
    post_norm = g.randn((d,), 1.0, w_std)
    wq = g.randn((d, d), 0.0, w_std)
    wk = g.randn((d, n_kv_heads * hd), 0.0, w_std)
    wv = g.randn((d, n_kv_heads * hd), 0.0, w_std)
    wo = g.randn((d, d), 0.0, w_std)
    w_router = g.randn((d, E), 0.0, w_std)
    gate, up, down = [], [], []
    for _ in range(n_shared + E):
        gate.append(g.randn((d, f), 0.0, w_std))
        up.append(g.randn((d, f), 0.0, w_std))
        down.append(g.randn((f, d), 0.0, w_std))
    rnd = round_bf16 if dtype == "bf16" else (lambda a: np.ascontiguousarray(a, np.float32))
    x, input_norm, post_norm = rnd(x), rnd(input_norm), rnd(post_norm)
    wq, wk, wv, wo, w_router = rnd(wq), rnd(wk), rnd(wv), rnd(wo), rnd(w_router)
    gate = [rnd(a) for a in gate]
    up = [rnd(a) for a in up]
    down = [rnd(a) for a in down]
    moe = MoEInputs(name=name + "-moe", T=T, d=d, f=f, E=E, k=k, n_shared=n_shared, dtype=dtype,
                    x=np.zeros((0, d), np.float32), w_router=w_router,
                    router_bias=np.zeros(E, np.float32), gate=gate, up=up, down=down)
    cos, sin = cos_sin if cos_sin is not None else rope_cache(max(seq_len, 1024), hd, rope_theta)
    return BlockInputs(name=name, batch=batch, seq_len=seq_len, d=d, n_heads=n_heads,
                       n_kv_heads=n_kv_heads, head_dim=hd, rope_theta=rope_theta, eps=1e-5,
                       dtype=dtype, x=x, input_norm=input_norm, post_norm=post_norm, wq=wq,
                       wk=wk, wv=wv, wo=wo, cos=cos, sin=sin, moe=moe)
