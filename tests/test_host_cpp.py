"""The C++ host mirror of GpuModelEngine (prichs_amd/host/gpu_model_engine.*)
through its C++ test program (tests/cpp/test_gpu_model_engine.cpp), which is
written like the reference's engine tests (crates/prichs-cuda/src/engine.rs:
2876-3182).

Both runs check prichs_host::load_checkpoint on a PRICHS02 file the program
writes byte by byte (model.rs:1648-1670).  The GPU test feeds it config-1
fixtures from the oracle: router logits within
1e-5, the stage-by-stage MoE (shared, then each expert on the oracle's token
lists, then finalize) and the fused device path within 1e-4 (f32).
"""
import os
import subprocess

import numpy as np
import pytest

from prichs_amd import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "test_gpu_model_engine")


def _run(args, timeout):
    assert os.path.exists(BIN), f"{BIN} is not built (run __graft_entry__.build())"
    r = subprocess.run([BIN, *args], capture_output=True, text=True, timeout=timeout)
    print(r.stdout, r.stderr, flush=True)
    return r


def _write_fixture(dirname, inp, ref):
    lines = []

    def put(kind, name, arr):
        a = np.ascontiguousarray(arr, dtype=np.float32 if kind == "f32" else np.int32)
        a.tofile(os.path.join(dirname, name + ".bin"))
        lines.append(f"{kind} {name} {a.size}")

    for key, val in (("T", inp.T), ("d", inp.d), ("f", inp.f), ("E", inp.E), ("k", inp.k)):
        lines.append(f"scalar {key} {val}")
    put("f32", "x", inp.x)
    # Expert j: 0 = the shared expert, 1.. = routed 0..E-1 (MoEInputs order).
    for j in range(inp.n_shared + inp.E):
        put("f32", f"gate{j}", inp.gate[j])
        put("f32", f"up{j}", inp.up[j])
        put("f32", f"down{j}", inp.down[j])
    put("f32", "w_router", inp.w_router)
    put("f32", "router_bias", inp.router_bias)
    put("f32", "logits", ref["logits"])
    put("f32", "out", ref["out"])
    put("i32", "offsets", ref["offsets"])
    put("i32", "row_token", ref["row_token"])
    put("f32", "row_weight", ref["row_weight"])
    with open(os.path.join(dirname, "manifest.txt"), "w") as fh:
        fh.write("\n".join(lines) + "\n")


def _has_gpu():
    import torch

    return torch.cuda.device_count() > 0


def test_engine_creation_without_device_raises():
    if _has_gpu():
        pytest.skip("a GPU is present: creation succeeds there (the GPU test covers it)")
    r = _run(["--no-gpu"], timeout=120)
    assert r.returncode == 0, r.stdout


@pytest.mark.gpu
def test_cpp_gpu_model_engine_mirror(orc, tmp_path):
    inp = synth.config_inputs(1)
    assert inp.n_shared == 1
    ref = orc.moe_forward(inp)
    _write_fixture(str(tmp_path), inp, ref)
    r = _run([str(tmp_path)], timeout=300)
    assert r.returncode == 0, r.stdout
    assert "PASSED: 0 failed" in r.stdout
