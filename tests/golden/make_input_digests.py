"""Writes tests/golden/input_sha256.json: the SHA-256 of every configuration's
synthetic inputs (prichs_amd/synth.py; configurations 1-4 MoEInputs.digest,
configuration 5 BlockInputs.digest), so that a change of the generator is
reported apart from kernel error.  bench.py prints the digest of the inputs it
ran on next to the committed one.

Run from the repository root:  python tests/golden/make_input_digests.py
"""
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from prichs_amd import synth  # noqa: E402


def digests() -> dict:
    out = {f"config{c}": synth.config_inputs(c).digest() for c in (1, 2, 3, 4)}
    out["config5"] = synth.make_block_inputs().digest()
    return out


def main():
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "input_sha256.json")
    with open(path, "w") as fh:
        json.dump(digests(), fh, indent=1, sort_keys=True)
        fh.write("\n")
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
