"""Writes the committed golden fixture of configuration 1 from the CPU oracle.

The reference holds no fixture that pins MoE-forward values, routing or the
permutation (its MoE test only asserts non-zero outputs,
crates/prichs-cuda/src/engine.rs:3067-3182), so this fixture records the
oracle's answer on the seeded config-1 inputs once; test_oracle.py pins the
oracle itself independently and then guards against drift with this file.

Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402
from prichs_amd import synth  # noqa: E402


def main():
    O.build()
    inp = synth.config_inputs(1)
    r = O.moe_forward(inp)
    rows = np.array([0, 1, 2, 3, 255, 256, 510, 511])
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "config1_oracle.npz")
    np.savez_compressed(
        out,
        input_sha256=np.array(inp.digest()),
        sel=r["sel"], gw=r["gw"], offsets=r["offsets"], row_token=r["row_token"],
        rows=rows, out_rows=r["out"][rows],
        out_abs_sum=np.array(float(np.abs(r["out"]).astype(np.float64).sum())),
    )
    print("wrote", out, "offsets", r["offsets"].tolist())


if __name__ == "__main__":
    main()
