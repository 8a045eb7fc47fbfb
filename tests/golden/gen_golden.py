"""Write tests/golden/golden.npz: the oracle's outputs for every case in
vectors.CASES plus the small model's greedy tokens.

Run from the repository root after building the oracle and the engine
library (the model case uses the engine's host-side weight generator):
    python tests/golden/gen_golden.py
"""
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [HERE, os.path.join(ROOT, "oracle"),
                os.path.join(ROOT, "enginesmith-qwen35-08b-long-decode-m5max-round005_amd")]

import numpy as np  # noqa: E402

import cases  # noqa: E402
import esdecode as E  # noqa: E402
import vectors as V  # noqa: E402


def main():
    out = {}
    for name, make in V.CASES.items():
        for key, val in cases.oracle_outputs(name, make()).items():
            out[f"{name}/{key}"] = val
    out["model/tokens"] = cases.oracle_model_tokens(E)
    path = os.path.join(HERE, "golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {len(out)} arrays, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
