#!/usr/bin/env python3
"""MoE-layer forward throughput on one MI355X (BASELINE.json metric).

A step is one full MoELayer forward (router + top-2, permutation, grouped
gate/up+SwiGLU GEMM, grouped down GEMM, combine) over one batch of synthetic
seeded tokens already resident in HBM.  Default workload: configuration 2
(T=8192, d=1536, f=1280, 1 shared + 8 routed experts, top-2, bf16 weights and
activations, fp32 accumulation).

Prints one JSON line.  `roofline` describes the dominant kernel (the grouped
gate/up GEMM), timed with HIP events on the launch stream over a pass of K
forwards; `cpu_baseline` times the CPU oracle (the reference algorithm
restated in C) on a bounded sample of the same workload on this host.

Order of the GPU passes: W warmup + K timed forwards from idle
(`value_first_pass`), about 30 ms of untimed forwards (the clock settles), K
forwards with stage events (per-kernel times, roofline), K forwards with the
caches flushed, copy references, and last W warmup + K timed forwards
(`value`).  The GPU clock takes tens of
milliseconds of sustained load to settle after idle, so the first pass
carries the ramp; `value` is the settled rate a serving loop sees.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "MoE-layer tokens/s + expert-GEMM TFLOP/s (% MFMA peak) at d=1536 top-2, 1 GPU"
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_F32_TFLOPS = 157.3    # MI355X fp32 matrix
PEAK_HBM_GBPS = 8000.0

WORKLOADS = {
    2: "config2: PRICHS-shape MoE layer forward, T=8192, d=1536, f=1280, 1 shared + 8 routed, "
       "top-2, bf16 weights/activations, fp32 accumulate",
    3: "config3: as config2 with T=16384 and router bias skewing ~60% of assignments to experts 0-1",
    4: "config4: decode-shape MoE layer forward, T=32, d=1536, f=1280, bf16",
    5: "config5: PrichsBlock forward (RMSNorm, GQA attention 12Q/3KV hd=128 with RoPE theta=500000, "
       "residual, RMSNorm, MoE d=1536 f=1280 1+8 top-2, residual), 4 x 2048 tokens, bf16",
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


FLUSH_BYTES = 512 << 20  # twice the 256 MB MALL: overwriting it evicts L2 and MALL


class Flusher:
    """Overwrites a 512 MiB device buffer (a fill kernel) so that the next
    kernel finds its inputs in HBM, not in L2 or the 256 MB MALL.  Run between
    event-timed repetitions, outside the timed intervals."""

    def __init__(self):
        import torch

        self.buf = torch.empty(FLUSH_BYTES // 4, dtype=torch.float32, device="cuda")

    def __call__(self):
        self.buf.zero_()


def timed_pass(step, steps: int, warmup: int) -> float:
    """W untimed warmup steps, then EXACTLY K timed steps bracketed by
    torch.cuda.synchronize() on both sides; returns the wall seconds of the K."""
    import torch

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    return time.perf_counter() - t0


# The GPU's clock ramps up over the first ~20 ms of sustained work after an
# idle spell (same box, config 2: the first 30 forwards after 10 warmup ones
# average 323 us, later ones 288 us), so K = 20 steps right after setup would
# time the ramp.  Each bench therefore runs W + K steps once from idle
# ("value_first_pass" in the line), about 30 ms of untimed steps, then its
# diagnostic passes (stage events, cache-flushed passes, the copy references
# -- all GPU work), then W warmup and the K timed steps that give `value`.
TIMING_NOTE = ("value: W warmup then K timed steps after the bench's diagnostic passes (GPU "
               "clock settled); value_first_pass: the same W + K straight after setup")


def settle(step, seconds_per_step: float, target_s: float = 0.03) -> int:
    """Untimed steps for about target_s of GPU work, so that the diagnostic
    passes that follow (the stage events behind the roofline) run at the
    settled clock the timed pass sees, not in the ramp after idle."""
    import torch

    n = int(min(2000, max(10, target_s / max(seconds_per_step, 1e-6))))
    for _ in range(n):
        step()
    torch.cuda.synchronize()
    return n


def device_caps():
    """CU count and peak clocks of the device (prichs_device_caps) and the bf16
    dense MFMA peak they imply (CUs x clock x 4096 FLOP/clk/CU: 4 SIMDs x one
    16x16x32 MFMA = 16384 FLOP per 16 cycles each)."""
    import ctypes as C

    from prichs_amd import _lib as L

    v = [C.c_int(0) for _ in range(4)]
    L.check(L.load().prichs_device_caps(*(C.byref(x) for x in v)))
    cus, clk, mclk, bus = (x.value for x in v)
    return {"compute_units": cus, "max_clock_MHz": clk / 1e3, "mem_clock_MHz": mclk / 1e3,
            "mem_bus_bits": bus,
            "bf16_dense_peak_TFLOPs_from_caps": cus * clk * 1e3 * 4096 / 1e12}


def _lib_copy(src, dst):
    from prichs_amd import ops

    ops.hbm_copy(src, dst)


def graph_event_ms(fn, reps: int = 20) -> float:
    """Mean device time of fn() over `reps` back-to-back calls, captured into
    one HIP graph and replayed between two events, so host launch overhead
    (Python and ctypes, ~10 us a call) cannot leave the GPU idle inside the
    interval -- short kernels would otherwise be timed at the host's pace."""
    import torch

    fn()  # one-time launch attributes stay outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    g.replay()
    b.record()
    torch.cuda.synchronize()
    del g
    return a.elapsed_time(b) / reps


def copy_bandwidth(reps: int = 10):
    """Device-to-device copy of 2 GiB with the library's streaming copy kernel
    (prichs_hbm_copy), timed with HIP events: read + write bytes per second,
    the measured practical HBM peak.  torch's copy of the same buffers is
    timed beside it for reference."""
    import torch

    n = (2 << 30) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    res = {}
    for name, fn in (("prichs_hbm_copy", lambda: _lib_copy(src, dst)),
                     ("torch_copy", lambda: dst.copy_(src))):
        for _ in range(2):
            fn()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / reps
        res[name] = {"GB/s": 2 * n * 4 / (ms * 1e-3) / 1e9, "ms": ms}
    del src, dst
    out = dict(res["prichs_hbm_copy"])
    out.update({"bytes_per_copy": 2 * n * 4, "torch_copy_GB/s": res["torch_copy"]["GB/s"],
                "kernel": "prichs_hbm_copy of 2 GiB (read + write counted), HIP events, mean of "
                          f"{reps}; torch_copy_GB/s: torch copy_ of the same buffers"})
    return out


def copy_same_bytes(moved_bytes: int, flush=None, reps: int = 10):
    """The practical roof of a memory-bound kernel that moves moved_bytes
    (reads + writes): the library's streaming copy (prichs_hbm_copy) of
    moved_bytes / 2, event-timed like the kernels -- warm (back to back), or
    with L2 and MALL flushed before each repetition when flush is given.  At
    tens of MB the ramp of a launch, not the 8 TB/s HBM peak, bounds any
    streaming kernel."""
    import torch

    n = max(4, (moved_bytes // 2 // 16) * 4)
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    _lib_copy(src, dst)
    if flush is None:  # warm: back-to-back copies in one graph
        ms = graph_event_ms(lambda: _lib_copy(src, dst), reps)
    else:  # each copy after a flush (the flush keeps the host ahead of the GPU)
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(reps)]
        for a, b in evs:
            flush()
            a.record()
            _lib_copy(src, dst)
            b.record()
        torch.cuda.synchronize()
        ms = sum(a.elapsed_time(b) for a, b in evs) / reps
    del src, dst
    return {"ms": ms, "GB/s": 2 * n * 4 / (ms * 1e-3) / 1e9}


def stage_vs_copy(ms: float, ms_flushed: float, nbytes: int, flush):
    """A memory-bound stage's rate against the library copy of the same bytes,
    warm and flushed: {"copy_same_bytes": .., "copy_same_bytes_flushed": ..,
    "frac_of_copy": .., "frac_of_copy_flushed": ..}."""
    warm = copy_same_bytes(nbytes)
    cold = copy_same_bytes(nbytes, flush)
    return {"copy_same_bytes": warm, "copy_same_bytes_flushed": cold,
            "frac_of_copy": warm["ms"] / ms, "frac_of_copy_flushed": cold["ms"] / ms_flushed}


def library_dense_equivalent(rows: int, d: int, f: int, reps: int = 50, rounds: int = 3):
    """Vendor-library yardstick for the expert GEMMs: torch.matmul (hipBLASLt)
    on one dense bf16 GEMM per expert GEMM with the same total rows and
    FLOPs -- [rows, d] x [d, 2f] for gate/up and [rows, f] x [f, d] for down,
    weights stored [N, K] as the packed expert weights are -- with no row
    gather, no ragged groups and no fused SwiGLU.  Event-timed: after 20
    warmup calls, `rounds` means of `reps` back-to-back calls; the best mean
    is reported (the library's run-to-run spread is large).  A measurement
    beside the product, never part of it."""
    import torch

    g = torch.Generator(device="cuda").manual_seed(0)
    out = {}
    for name, (m, n, kk) in (("gate_up", (rows, 2 * f, d)), ("down", (rows, d, f))):
        a = torch.randn(m, kk, device="cuda", dtype=torch.bfloat16, generator=g)
        w = torch.randn(n, kk, device="cuda", dtype=torch.bfloat16, generator=g)
        c = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
        for _ in range(20):
            torch.matmul(a, w.t(), out=c)
        means = []
        for _ in range(rounds):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                torch.matmul(a, w.t(), out=c)
            e1.record()
            torch.cuda.synchronize()
            means.append(e0.elapsed_time(e1) / reps)
        ms = min(means)
        tf = 2.0 * m * n * kk / (ms * 1e-3) / 1e12
        out[name] = {"shape_MNK": [m, n, kk], "ms": ms, "TFLOP/s": tf,
                     "frac_of_peak": tf / PEAK_BF16_TFLOPS, "ms_round_means": means}
        del a, w, c
    tot = out["gate_up"]["ms"] + out["down"]["ms"]
    out["both"] = {"ms": tot, "TFLOP/s": 6.0 * rows * d * f / (tot * 1e-3) / 1e12,
                   "frac_of_peak": 6.0 * rows * d * f / (tot * 1e-3) / 1e12 / PEAK_BF16_TFLOPS}
    out["library"] = f"torch {torch.__version__} matmul (hipBLASLt), bf16 in/out, fp32 accumulate"
    return out


def committed_digest(name: str):
    try:
        with open(os.path.join(ROOT, "tests", "golden", "input_sha256.json")) as fh:
            return json.load(fh).get(name)
    except OSError:
        return None


def inputs_record(name: str, digest: str):
    want = committed_digest(name)
    return {"sha256": digest, "committed_sha256": want, "matches_committed": digest == want}


def cpu_model() -> str:
    """The host CPU's model name (Linux /proc/cpuinfo), or "unknown"."""
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def one_thread(run, n: int, unit_tokens: int):
    """run(n) on one oracle thread (the rest of the baseline uses all of them)."""
    from oracle import oracle

    cores = oracle.num_threads()
    oracle.set_num_threads(1)
    try:
        t = run(n)
    finally:
        oracle.set_num_threads(cores)
    return {"value": unit_tokens / t, "unit": "tokens/s", "cores": 1,
            "sample": f"first {n} tokens, {t:.2f} s"}


def cpu_baseline(inp, target_s: float):
    """Times the CPU oracle on a token sample sized to about target_s seconds."""
    import numpy as np

    from oracle import oracle
    from prichs_amd import synth

    oracle.build()
    cores = oracle.num_threads()

    def run(n):
        sub = synth.MoEInputs(**{**inp.__dict__, "x": inp.x[:n], "T": n})
        t0 = time.perf_counter()
        oracle.moe_forward(sub)
        return time.perf_counter() - t0

    n0 = min(inp.T, 64)
    t = run(n0)
    n = int(min(inp.T, max(n0, n0 * target_s / max(t, 1e-3))))
    n = max(n0, n - n % 64) if n >= 64 else n
    t = run(n)
    return {
        "value": n / t, "unit": "tokens/s", "cores": cores, "kind": "port",
        "sample": f"first {n} of {inp.T} tokens of the same synthetic inputs; C oracle "
                  f"(reference CPU algorithm: naive k-outer f32 GEMM, serial gating/binning/"
                  f"scatter), OpenMP over rows on {cores} threads, {t:.1f} s",
        "seconds": t,
        "cpu_model": cpu_model(),
        "one_thread": one_thread(run, n0, n0),
    }


def cold_weights_pass(eng, inp, x, args, layers=4):
    """The layer's rate when its weights are not resident in the 256 MB MALL:
    `layers` engines with distinct weights (layer l: the same synthetic
    tensors rolled by l along their columns, so equally distributed but held
    apart in HBM; 4 x 106 MB at config 2) run one after another on the same
    x, W + K such rounds timed as in the headline pass, after it.  Reported
    beside `value`, not as it."""
    import numpy as np
    import torch

    from prichs_amd import moe

    log(f"bench: cold-weights pass, {layers} layers with distinct weights")
    engines = [eng]
    for l in range(1, layers):
        e = moe.MoEEngine(inp.d, inp.f, inp.E, inp.k, inp.n_shared, inp.dtype, max_tokens=inp.T)
        roll = lambda a: np.roll(a, l, axis=1)  # noqa: E731
        e.upload(np.roll(inp.w_router, l, axis=0), inp.router_bias, [roll(a) for a in inp.gate],
                 [roll(a) for a in inp.up], [roll(a) for a in inp.down])
        engines.append(e)
    outs = [torch.empty((inp.T, inp.d), dtype=x.dtype, device="cuda") for _ in engines]

    def rounds():
        for e, o in zip(engines, outs):
            e.forward(x, out=o)

    elapsed = timed_pass(rounds, args.steps, args.warmup)
    for e in engines[1:]:
        e.close()
    per_layer = elapsed / args.steps / layers
    return {"layers": layers, "tokens/s": inp.T / per_layer, "ms_per_layer": per_layer * 1e3,
            "weights_MB_per_layer": round(sum(a.size for a in (*inp.gate, *inp.up, *inp.down))
                                          * 2 / 1e6, 1),
            "note": "each layer's weights evicted from the MALL by the other layers' between "
                    "its forwards; layers 1.. use the same synthetic weights rolled along their "
                    "columns (distinct tensors in HBM); x stays resident"}


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=2, choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--backward", action="store_true",
                    help="time a training step instead (the forward plus the MoE backward, "
                         "prichs_moe_engine_backward) on configuration 2 or 3")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run 3 plain device copies of 1 GiB (known bytes) so that "
                         "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE can be scaled")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (--gpus {args.gpus} requested): the MoE hot path "
              "is built and measured on a single MI355X; multi-GPU sharding is design-only.",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from prichs_amd import moe, synth

    if args.copy_calibration:
        copy_calibration()
    if args.config == 5:
        return bench_block(args)
    if args.backward:
        return bench_backward(args)
    log(f"bench: generating config {args.config} inputs")
    inp = synth.config_inputs(args.config)
    T, d, f, E, k, S = inp.T, inp.d, inp.f, inp.E, inp.k, inp.n_shared
    eng = moe.MoEEngine(d, f, E, k, S, inp.dtype, max_tokens=T)
    eng.upload(inp.w_router, inp.router_bias, inp.gate, inp.up, inp.down)
    x = torch.from_numpy(inp.x).to("cuda").to(torch.bfloat16 if inp.dtype == "bf16" else torch.float32)
    out = torch.empty((T, d), dtype=x.dtype, device="cuda")
    def fwd():
        eng.forward(x, out=out)

    # Throughput over K forwards with nothing else on the stream (first from
    # idle, then again after the diagnostics); in between, the same K
    # forwards with the engine's stage events (HIP events on its launch
    # stream between the stages), which give the per-kernel times and the
    # roofline.  Six events per forward cost ~3.5 us each on the stream, a
    # third of a decode-sized forward, so they stay out of `value`.
    log(f"bench: first pass, {args.warmup} warmup + {args.steps} timed steps")
    elapsed_first = timed_pass(fwd, args.steps, args.warmup)
    n_settle = settle(fwd, elapsed_first / args.steps)
    eng.set_timing(args.steps)
    for _ in range(args.steps):
        eng.forward(x, out=out)
    torch.cuda.synchronize()
    ms = eng.stage_ms()
    # The same forwards with L2 and the MALL flushed before each one (the
    # flush sits between forwards, outside every stage interval): the
    # router reads x from HBM as a layer does after the attention sub-layer.
    flush = Flusher()
    eng.set_timing(args.steps)
    for _ in range(args.steps):
        flush()
        eng.forward(x, out=out)
    torch.cuda.synchronize()
    ms_cold = eng.stage_ms()
    eng.set_timing(0)
    es_ = 2 if inp.dtype == "bf16" else 4
    copy_ref = {
        "router": stage_vs_copy(ms["router"], ms_cold["router"],
                                T * d * es_ + d * E * 4 + T * E * 4 + T * k * 8, flush),
        "combine": stage_vs_copy(ms["combine"], ms_cold["combine"],
                                 (T * k + S * T) * d * es_ + T * k * 12 + T * d * es_, flush)}
    del flush
    # Library yardstick (prefill bf16 shapes only; decode is HBM-bound).
    rows_ = T * k + S * T
    lib = (library_dense_equivalent(rows_, d, f)
           if inp.dtype == "bf16" and T * k >= 64 * E else None)
    # The cold-weights rate (before the timing pass, whose W warmup forwards
    # bring the layer's weights back into the MALL, so that the timing pass
    # stays the run's last one).
    cold = cold_weights_pass(eng, inp, x, args) if T * k >= 64 * E else None
    log(f"bench: timing pass, {args.warmup} warmup + {args.steps} timed steps")
    elapsed = timed_pass(fwd, args.steps, args.warmup)
    log("bench: stage ms", json.dumps({kk: round(v, 4) for kk, v in ms.items()}))
    log("bench: stage ms (flushed)", json.dumps({kk: round(v, 4) for kk, v in ms_cold.items()}))

    es = 2 if inp.dtype == "bf16" else 4
    rows = T * k + S * T
    flops_gate_up = 4.0 * d * f * rows
    flops_down = 2.0 * d * f * rows
    peak = PEAK_BF16_TFLOPS if inp.dtype == "bf16" else PEAK_F32_TFLOPS
    t_gu = ms["gate_up"] / 1e3
    t_dn = ms["down"] / 1e3
    gu_tflops = flops_gate_up / t_gu / 1e12
    gemm_tflops = (flops_gate_up + flops_down) / (t_gu + t_dn) / 1e12
    router_bytes = T * d * es + d * E * 4 + T * E * 4 + T * k * 8
    permute_bytes = T * k * 8 + (T * k + T) * 4 + T * k * 8
    combine_bytes = rows * d * es + T * k * 12 + T * d * es

    def gbps(b, stage, m=ms):
        return b / (m[stage] / 1e3) / 1e9 if m[stage] > 0 else None

    kernel = "grouped gate/up GEMM + fused SwiGLU (bf16_gemm_kernel<Bf16Cfg<256,256,4,2>, Bf16Cfg<256,256,4,2>, true>)"
    # The engine's decode path (bf16, 4 < E <= 8, one shared expert, T <= 32,
    # d % 128 == 0, f % 64 == 0; config 4 meets it).
    decode = (inp.dtype == "bf16" and S == 1 and 4 < E <= 8 and T <= 32 and d % 128 == 0
              and f % 64 == 0)
    if T * k < 64 * E:  # fewer than 64 rows per routed expert on average
        # Decode shape: every touched expert's gate/up weights are streamed once
        # for a handful of rows, so the launch is bound by HBM, not MFMA.  When
        # one router workgroup covers the batch (T <= 32 here) the engine runs
        # the router inside a gate/up launch over every token of every expert:
        # all E + S experts' weights, x, and the activations of G T rows.
        sel = eng.stash()["selected_experts"].cpu().numpy()
        touched = len(set(sel.reshape(-1).tolist())) + S
        if decode:
            gu_bytes = (E + S) * d * 2 * f * es + T * d * es + (E + S) * T * f * es
            kernel = ("router workgroup + dense gate/up GEMM + fused SwiGLU, decode launch "
                      "(skinny::decode_gate_up_router_kernel<4>)")
        else:
            gu_bytes = touched * d * 2 * f * es + rows * d * es + rows * f * es
            kernel = "grouped gate/up GEMM + fused SwiGLU, decode shape (skinny::skinny_gemm_kernel<true, 4, 1>)"
        bw = gu_bytes / t_gu / 1e9
        tfile = "pmc_config4_decode_traffic.txt"
        roofline = {"kernel": kernel, "bound": "hbm", "achieved": bw, "peak": PEAK_HBM_GBPS,
                    "unit": "GB/s", "frac": bw / PEAK_HBM_GBPS,
                    "traffic": measured_traffic(tfile, "gate_up") if args.config == 4 else None,
                    "traffic_source": f"profiles/{tfile} (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE, "
                                      "copy-calibrated)" if args.config == 4 else None,
                    "algorithmic_bytes_per_launch": gu_bytes, "experts_touched": touched,
                    "avg_launch_ms": ms["gate_up"],
                    "timed_over": "HIP events on the engine's launch stream between the stages, "
                                  f"over a pass of the same K forwards after {n_settle} untimed "
                                  "settling forwards"}
    else:
        roofline = {
            "kernel": kernel, "bound": "mfma", "achieved": gu_tflops, "peak": peak,
            "unit": "TFLOP/s", "frac": gu_tflops / peak,
            "traffic": measured_traffic("pmc_config2_traffic.txt", "gate_up") if args.config == 2 else None,
            "traffic_source": "profiles/pmc_config2_traffic.txt (rocprofv3 --pmc FETCH_SIZE, "
                              "WRITE_SIZE, copy-calibrated)" if args.config == 2 else None,
            "mfma_busy_source": "profiles/pmc_config2_mfma.txt (SQ_VALU_MFMA_BUSY_CYCLES)"
                                if args.config == 2 else None,
            "algorithmic_flops_per_launch": flops_gate_up,
            "avg_launch_ms": ms["gate_up"],
            "timed_over": "HIP events on the engine's launch stream between the stages, over a "
                          f"pass of the same K forwards after {n_settle} untimed settling forwards",
        }

    res = {
        "metric": METRIC,
        "value": T * args.steps / elapsed,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": elapsed / args.steps * 1e3,
        "value_first_pass": T * args.steps / elapsed_first,
        "timing_note": TIMING_NOTE,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": inp.dtype,
        "data": "synthetic (seeded SplitMix64 + Box-Muller, seed 0)",
        "config": {"workload": WORKLOADS[args.config], "tokens": T, "d_model": d, "d_ffn": f,
                   "routed_experts": E, "shared_experts": S, "top_k": k},
        "roofline": roofline,
        "expert_gemm": {"tflops": gemm_tflops, "frac_of_peak": gemm_tflops / peak,
                        "gate_up_ms": ms["gate_up"], "down_ms": ms["down"],
                        "down_tflops": flops_down / t_dn / 1e12,
                        "library_dense_same_flops": lib},
        "memory_bound_stages": {
            "router": {"ms": ms["router"], "GB/s": gbps(router_bytes, "router"),
                       "ms_flushed": ms_cold["router"],
                       "GB/s_flushed": gbps(router_bytes, "router", ms_cold), "bytes": router_bytes,
                       **copy_ref["router"]},
            "permute": {"ms": ms["permute"], "GB/s": gbps(permute_bytes, "permute"),
                        "ms_flushed": ms_cold["permute"],
                        "GB/s_flushed": gbps(permute_bytes, "permute", ms_cold),
                        "bytes": permute_bytes},
            "combine": {"ms": ms["combine"], "GB/s": gbps(combine_bytes, "combine"),
                        "ms_flushed": ms_cold["combine"],
                        "GB/s_flushed": gbps(combine_bytes, "combine", ms_cold),
                        "bytes": combine_bytes, **copy_ref["combine"]},
            "peak_GB/s": PEAK_HBM_GBPS,
            "note": "flushed = L2 and MALL overwritten (512 MiB) before each forward, outside the "
                    "stage intervals; the combine reads y right after the down GEMM wrote it, with "
                    "non-temporal loads (y is dead afterwards, so it leaves the caches to the "
                    "weights of the next forward; the combine itself is slower for it); "
                    "copy_same_bytes* = the library's streaming copy (prichs_hbm_copy) of the "
                    "stage's bytes, timed the same way; frac_of_copy = copy ms / stage ms",
        },
        "stage_ms": {kk: v for kk, v in ms.items() if kk != "n"},
        "stage_ms_flushed": {kk: v for kk, v in ms_cold.items() if kk != "n"},
        **({"stage_note": "decode path: the router and the permutation run inside the gate/up "
                          "launch (its first workgroup), so the router and permute intervals hold "
                          "no kernel, only the gap between event records; gate_up times the "
                          "router + gate/up launch"} if decode else {}),
        **({"cold_weights": cold} if cold is not None else {}),
        "inputs": inputs_record(f"config{args.config}", inp.digest()),
        "device": torch.cuda.get_device_name(0),
        "device_caps": device_caps(),
        "copy_bandwidth": copy_bandwidth(),
    }
    if not args.no_cpu_baseline:
        log("bench: CPU baseline (oracle)")
        res["cpu_baseline"] = cpu_baseline(inp, args.cpu_seconds)
    else:
        res["cpu_baseline"] = None
    eng.close()
    print(json.dumps(res), flush=True)


TRAIN_METRIC = ("MoE-layer training step (forward + backward) tokens/s + backward GEMM TFLOP/s "
                "at d=1536 top-2, 1 GPU")


def cpu_baseline_train(inp, d_out, target_s: float):
    """Times the CPU oracle's forward + backward on a token sample of about target_s."""
    from oracle import oracle
    from prichs_amd import synth

    oracle.build()
    cores = oracle.num_threads()

    def run(n):
        sub = synth.MoEInputs(**{**inp.__dict__, "x": inp.x[:n], "T": n})
        t0 = time.perf_counter()
        oracle.moe_forward(sub)
        oracle.moe_backward(sub, d_out[:n], dx_weighting=2)
        return time.perf_counter() - t0

    n0 = min(inp.T, 32)
    t = run(n0)
    n = int(min(inp.T, max(n0, n0 * target_s / max(t, 1e-3))))
    n = max(n0, n - n % 32)
    t = run(n)
    return {
        "value": n / t, "unit": "tokens/s", "cores": cores, "kind": "port",
        "sample": f"first {n} of {inp.T} tokens of the same synthetic inputs; C oracle forward "
                  f"+ backward (reference CPU algorithm, f32, naive GEMMs), OpenMP over rows on "
                  f"{cores} threads, {t:.1f} s",
        "seconds": t,
        "cpu_model": cpu_model(),
        "one_thread": one_thread(run, n0, n0),
    }


def bench_backward(args):
    """One step = MoELayer forward + the MoE backward (d_x and every weight
    gradient, accumulated into f32 buffers in the reference's parameter
    layout) on configuration 2 (or 3)."""
    import numpy as np
    import torch

    from prichs_amd import moe, synth

    cfg = args.config if args.config in (2, 3) else 2
    log(f"bench: generating config {cfg} inputs (training step)")
    inp = synth.config_inputs(cfg)
    T, d, f, E, k = inp.T, inp.d, inp.f, inp.E, inp.k
    G = 1 + E
    eng = moe.MoEEngine(d, f, E, k, 1, inp.dtype, max_tokens=T)
    eng.enable_backward()
    eng.upload(inp.w_router, inp.router_bias, inp.gate, inp.up, inp.down)
    bf = torch.bfloat16
    x = torch.from_numpy(inp.x).to("cuda").to(bf)
    d_out_np = synth.round_bf16(np.random.default_rng(1).standard_normal((T, d)).astype(np.float32))
    d_out = torch.from_numpy(d_out_np).to("cuda").to(bf)
    out = torch.empty((T, d), dtype=bf, device="cuda")
    d_x = torch.empty((T, d), dtype=bf, device="cuda")
    grads = {"d_router": torch.zeros((d, E), dtype=torch.float32, device="cuda"),
             "flat": torch.zeros((G, 3, d * f), dtype=torch.float32, device="cuda")}

    # beta = 0: the gradients are overwritten, as zero_grads() followed by the
    # backward (forward_backward_vram, model.rs:1198-1207) leaves them.
    def step():
        eng.forward(x, out=out)
        eng.backward(x, d_out, grads, dx_weighting=2, d_x=d_x, beta=0)

    # Throughput without events (first from idle, then again after the
    # event pass), and in between the same steps with the engine's stage
    # events for the per-kernel times (as in the forward bench).
    log(f"bench: first pass, {args.warmup} warmup + {args.steps} timed training steps")
    elapsed_first = timed_pass(step, args.steps, args.warmup)
    n_settle = settle(step, elapsed_first / args.steps)
    eng.set_timing(args.steps)
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    fms = eng.stage_ms()
    bms = eng.backward_stage_ms()
    eng.set_timing(0)
    log(f"bench: timing pass, {args.warmup} warmup + {args.steps} timed training steps")
    elapsed = timed_pass(step, args.steps, args.warmup)
    log("bench: forward stage ms", json.dumps({kk: round(v, 4) for kk, v in fms.items()}))
    log("bench: backward stage ms", json.dumps({kk: round(v, 4) for kk, v in bms.items()}))

    rows = T * (k + 1)
    np_gu = 2 * ((f + 31) // 32 * 32)
    np_gu = (np_gu + 255) // 256 * 256
    # Algorithmic flops per launch (padding excluded).  The gate/up
    # pre-activations come from the forward's GEMM, so the backward has four.
    gemm_flops = {
        "dw_down": 2.0 * rows * f * d, "d_act": 2.0 * rows * d * f,
        "dw_gate_up": 4.0 * rows * d * f, "d_x_gemm": 4.0 * rows * f * d,
    }
    kernels = {
        "dw_down": "grouped weight gradient dW_down += act^T dY (wgrad_bf16_kernel<false>, then wgrad_reduce_kernel<false>; the stage times both)",
        "d_act": "grouped GEMM dA = dY Wd^T with the SwiGLU backward in its epilogue (bf16_gemm_kernel<Bf16Cfg<256,256,4,2>, Bf16Cfg<256,128,4,2>, false, true>: dG, dU into the pre-activations in place; the stage and its TFLOP/s include that memory-bound work)",
        "dw_gate_up": "grouped weight gradient dW_gate/up += x^T [dG dU] (wgrad_bf16_kernel<true>, then wgrad_reduce_kernel<true> adding the shared expert's K-chunk partials; the stage times both)",
        "d_x_gemm": "grouped GEMM dX = [dG dU] [Wg Wu]^T (bf16_gemm_kernel<Bf16Cfg<256,256,4,2>, Bf16Cfg<256,128,4,2>, false>)",
    }
    per = {kk: {"ms": bms[kk], "tflops": fl / (bms[kk] / 1e3) / 1e12}
           for kk, fl in gemm_flops.items()}
    dom = max(per, key=lambda kk: per[kk]["ms"])
    bwd_gemm_ms = sum(bms[kk] for kk in gemm_flops)
    bwd_gemm_tflops = sum(gemm_flops.values()) / (bwd_gemm_ms / 1e3) / 1e12
    es = 2
    swiglu_bytes = rows * np_gu * es * 2 + rows * f * es
    combine_bytes = rows * d * es + T * k * 16 + T * d * es + T * E * 4 + d * E * 4

    def gbps(b, stage):
        return b / (bms[stage] / 1e3) / 1e9 if bms[stage] > 0 else None

    # The SwiGLU backward runs inside the dA GEMM (bf16 at tiled sizes): its
    # own interval then holds only its two events.  The same condition makes
    # the rows pass cover the routed rows only (the shared expert's dY and xg
    # rows are d_out and x, read in place by their consumers).
    swiglu_fused = bms["swiglu_bwd"] < 0.2 * bms["d_act"]
    # One wave per token: d_out[t] and x[t] read once; dY and xg written and
    # (routed) y read per row.
    rows_pass = T * k if swiglu_fused else rows
    rows_bytes = T * d * es * 2 + rows_pass * d * es * 2 + T * k * d * es + T * k * 8

    res = {
        "metric": TRAIN_METRIC,
        "value": T * args.steps / elapsed,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": elapsed / args.steps * 1e3,
        "value_first_pass": T * args.steps / elapsed_first,
        "timing_note": TIMING_NOTE,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": inp.dtype,
        "data": "synthetic (seeded SplitMix64 + Box-Muller, seed 0; d_out numpy seed 1)",
        "config": {"workload": WORKLOADS[cfg].replace("forward", "forward + backward"),
                   "tokens": T, "d_model": d, "d_ffn": f, "routed_experts": E,
                   "shared_experts": 1, "top_k": k, "dx_weighting": 2,
                   "grads": "f32, reference parameter layout, overwritten (beta = 0: zero_grads "
                            "then the backward)"},
        "roofline": {"kernel": kernels[dom], "bound": "mfma", "achieved": per[dom]["tflops"],
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": per[dom]["tflops"] / PEAK_BF16_TFLOPS, "traffic": None,
                     "algorithmic_flops_per_launch": gemm_flops[dom],
                     "avg_launch_ms": per[dom]["ms"],
                     "timed_over": "HIP events on the engine's launch stream between the stages, "
                                   f"over K training steps after {n_settle} untimed settling steps"},
        "backward_gemms": {"tflops": bwd_gemm_tflops, "frac_of_peak": bwd_gemm_tflops / PEAK_BF16_TFLOPS,
                           "per_stage": per},
        "memory_bound_stages": {
            "rows": {"ms": bms["rows"], "GB/s": gbps(rows_bytes, "rows"), "bytes": rows_bytes},
            "swiglu_bwd": ({"ms": bms["swiglu_bwd"], "fused_into": "d_act", "GB/s": None,
                            "bytes": swiglu_bytes} if swiglu_fused else
                           {"ms": bms["swiglu_bwd"], "GB/s": gbps(swiglu_bytes, "swiglu_bwd"),
                            "bytes": swiglu_bytes}),
            "combine": {"ms": bms["combine"], "GB/s": gbps(combine_bytes, "combine"),
                        "bytes": combine_bytes},
            "peak_GB/s": PEAK_HBM_GBPS,
        },
        "forward_ms": fms["total"],
        "backward_ms": bms["total"],
        "backward_stage_ms": {kk: v for kk, v in bms.items() if kk != "n"},
        "inputs": inputs_record(f"config{cfg}", inp.digest()),
        "device": torch.cuda.get_device_name(0),
        "device_caps": device_caps(),
    }
    if not args.no_cpu_baseline:
        log("bench: CPU baseline (oracle forward + backward)")
        res["cpu_baseline"] = cpu_baseline_train(inp, d_out_np, args.cpu_seconds)
    else:
        res["cpu_baseline"] = None
    eng.close()
    print(json.dumps(res), flush=True)


COPY_BYTES = 1 << 30


def copy_calibration():
    """Three device-to-device copies of exactly COPY_BYTES with the library's
    streaming copy kernel (prichs_hbm_copy: reads and writes each byte once,
    so its FETCH_SIZE / WRITE_SIZE per dispatch should read COPY_BYTES)."""
    import torch

    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        _lib_copy(src, dst)
    torch.cuda.synchronize()
    log(f"bench: copy calibration, 3 x {COPY_BYTES} bytes")
    del src, dst


def measured_traffic(name, kernel):
    """HBM-side bytes per launch of `kernel` from a committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, each scaled by the copy calibration:
    the line traffic_bytes_per_launch[kernel] = ...), or None."""
    path = os.path.join(ROOT, "profiles", name)
    key = f"traffic_bytes_per_launch[{kernel}]"
    try:
        with open(path) as fh:
            for line in fh:
                if line.startswith(key):
                    return float(line.split("=")[1].split()[0])
    except OSError:
        return None
    return None


def bench_block(args):
    """Config 5: one PrichsBlock forward per step (tokens/s), with the attention
    kernel timed on its own over the same rows (causal TFLOP/s)."""
    import numpy as np
    import torch

    from prichs_amd import block, ops, synth

    log("bench: generating config 5 inputs")
    inp = synth.make_block_inputs()
    B, S, d = inp.batch, inp.seq_len, inp.d
    T = B * S
    blk = block.PrichsBlock.from_inputs(inp)
    eng = blk.engine
    x = torch.from_numpy(inp.x).to("cuda").to(torch.bfloat16)
    out = torch.empty((T, d), dtype=torch.bfloat16, device="cuda")
    def fwd():
        eng.forward(x, B, S, out=out)

    elapsed_first = timed_pass(fwd, args.steps, args.warmup)
    # Attention alone, as the block runs it: on the last forward's stashed
    # q/k/v (q as projected, k rotated) through the entry point that rotates q
    # as it loads it, with the block's RoPE tables; HIP events on the stream.
    qkv = eng.stash()["qkv"]
    Hq, Hkv, hd = inp.n_heads, inp.n_kv_heads, inp.head_dim
    q, k, v = qkv[:, :Hq * hd], qkv[:, Hq * hd:(Hq + Hkv) * hd], qkv[:, (Hq + Hkv) * hd:]
    cos, sin = (torch.from_numpy(np.ascontiguousarray(a, np.float32)).to("cuda")
                for a in synth.rope_cache(S, hd, inp.rope_theta))
    ao = torch.empty((T, d), dtype=torch.bfloat16, device="cuda")
    att_fn = lambda: ops.attention(q, k, v, B, S, Hq, Hkv, out=ao, rope_q=(cos, sin, 0))  # noqa: E731
    for _ in range(3):
        att_fn()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        att_fn()
    e1.record()
    torch.cuda.synchronize()
    att_ms = e0.elapsed_time(e1) / args.steps

    def event_ms(fn, reps=max(args.steps, 20)):
        # back-to-back calls replayed from a graph (no host gaps)
        return graph_event_ms(fn, reps)

    flush = Flusher()

    def event_ms_flushed(fn, reps=args.steps):
        # One event pair per repetition with L2 and the MALL flushed before
        # it, outside the pair: the kernel reads its inputs from HBM.
        for _ in range(3):
            fn()
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(reps)]
        for a, b in evs:
            flush()
            a.record()
            fn()
            b.record()
        torch.cuda.synchronize()
        return sum(a.elapsed_time(b) for a, b in evs) / reps

    # HBM-bound sub-layers alone at the block's shapes: RMSNorm of x [T, d]
    # (bf16 in/out, f32 weight) and RoPE in place on Q [T, 12, 128] and K [T, 3, 128].
    w_norm = torch.from_numpy(np.ascontiguousarray(inp.input_norm, np.float32)).to("cuda")
    rn_out = torch.empty_like(x)
    rn_ms = event_ms(lambda: ops.rmsnorm(x, w_norm, want_rstd=False, out=rn_out))
    rn_ms_cold = event_ms_flushed(lambda: ops.rmsnorm(x, w_norm, want_rstd=False, out=rn_out))
    qr = q.contiguous().view(B, S, Hq, hd)
    kr = k.contiguous().view(B, S, Hkv, hd)
    rope_fn = lambda: (ops.rope_(qr, cos, sin, S, B, S), ops.rope_(kr, cos, sin, S, B, S))  # noqa: E731
    rope_ms = event_ms(rope_fn)
    rope_ms_cold = event_ms_flushed(rope_fn)
    rn_bytes = 2 * T * d * 2 + d * 4
    rope_bytes = 2 * T * (Hq + Hkv) * hd * 2 + 2 * S * (hd // 2) * 4
    rn_copy = stage_vs_copy(rn_ms, rn_ms_cold, rn_bytes, flush)
    rope_copy = stage_vs_copy(rope_ms, rope_ms_cold, rope_bytes, flush)
    del flush
    elapsed = timed_pass(fwd, args.steps, args.warmup)
    att_flops = B * Hq * 4.0 * hd * S * (S + 1) / 2  # causal QK^T + PV
    moe_flops = 6.0 * d * inp.moe.f * T * (inp.moe.k + 1)
    proj_flops = 2.0 * T * d * (d + 2 * Hkv * hd) + 2.0 * T * d * d
    ms = elapsed / args.steps * 1e3
    res = {
        "metric": "PrichsBlock forward tokens/s (config 5)",
        "value": T * args.steps / elapsed, "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms,
        "value_first_pass": T * args.steps / elapsed_first, "timing_note": TIMING_NOTE,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded SplitMix64 + Box-Muller, seed 0)",
        "config": {"workload": WORKLOADS[5], "batch": B, "seq_len": S, "d_model": d},
        "roofline": {"kernel": "attn_fwd_kernel (causal GQA flash attention, q rotated by RoPE "
                               "as it is loaded, as in the block)", "bound": "mfma",
                     "achieved": att_flops / (att_ms * 1e-3) / 1e12, "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": att_flops / (att_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
                     "traffic": None, "algorithmic_flops_per_launch": att_flops,
                     "avg_launch_ms": att_ms},
        "block_tflops": (att_flops + moe_flops + proj_flops) / (ms * 1e-3) / 1e12,
        "memory_bound_stages": {
            "rmsnorm": {"ms": rn_ms, "GB/s": rn_bytes / (rn_ms * 1e-3) / 1e9,
                        "ms_flushed": rn_ms_cold,
                        "GB/s_flushed": rn_bytes / (rn_ms_cold * 1e-3) / 1e9, "bytes": rn_bytes,
                        **rn_copy},
            "rope_q_and_k": {"ms": rope_ms, "GB/s": rope_bytes / (rope_ms * 1e-3) / 1e9,
                             "ms_flushed": rope_ms_cold,
                             "GB/s_flushed": rope_bytes / (rope_ms_cold * 1e-3) / 1e9,
                             "bytes": rope_bytes,
                             **rope_copy,
                             "note": "two launches (Q 12 heads, K 3 heads); the copy is one"},
            "peak_GB/s": PEAK_HBM_GBPS,
            "note": "flushed = L2 and MALL overwritten (512 MiB) before each repetition, outside "
                    "its event pair; copy_same_bytes* = the library's streaming copy "
                    "(prichs_hbm_copy) of the stage's bytes, timed the same way; frac_of_copy = "
                    "copy ms / stage ms",
        },
        "inputs": inputs_record("config5", inp.digest()),
        "device": torch.cuda.get_device_name(0),
        "device_caps": device_caps(),
        "copy_bandwidth": copy_bandwidth(),
    }
    eng.close()
    if not args.no_cpu_baseline:
        log("bench: CPU baseline (oracle block forward)")
        res["cpu_baseline"] = cpu_baseline_block(inp, args.cpu_seconds)
    else:
        res["cpu_baseline"] = None
    print(json.dumps(res), flush=True)


def cpu_baseline_block(inp, target_s: float):
    """Times the CPU oracle's block forward on a prefix of the first sequence:
    with causal attention a prefix's rows need no later rows, so the prefix is
    an exact sample of the workload.  The prefix doubles (from 64 rows) until a
    run takes a third of target_s or the whole sequence is covered."""
    import dataclasses

    from oracle import oracle

    oracle.build()
    cores = oracle.num_threads()

    def run(n):
        sub = dataclasses.replace(inp, batch=1, seq_len=n, x=inp.x[:n])
        t0 = time.perf_counter()
        oracle.block_forward(sub)
        return time.perf_counter() - t0

    n = 64
    t = run(n)
    while t < target_s / 3 and n < inp.seq_len:
        n = min(inp.seq_len, 2 * n)
        t = run(n)
    note = ("" if n == inp.seq_len else
            "; a prefix's tokens attend to fewer keys than the average token of a full sequence")
    return {
        "value": n / t, "unit": "tokens/s", "cores": cores, "kind": "port",
        "sample": f"first {n} rows of sequence 0 (of {inp.batch} x {inp.seq_len}); C oracle block "
                  f"forward (RMSNorm, f32 projections, causal GQA attention with RoPE, MoE, "
                  f"residuals), OpenMP over rows on {cores} threads, {t:.1f} s{note}",
        "seconds": t,
        "cpu_model": cpu_model(),
        "one_thread": one_thread(run, 64, 64),
    }


if __name__ == "__main__":
    main()
