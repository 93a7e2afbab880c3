"""Writes tests/golden/oracle_small.npz: small seeded Q4_0 / Q8_0 weights and
activations with the oracle's dequantized weights and fp64 outputs.

The reference (Rust) cannot run here, so these vectors come from the oracle,
which tests/test_oracle.py pins against the reference's own known answers first;
they guard the oracle and the GPU path against regressions.  Re-run only when
the synthetic-input definition changes:

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "openmini-v1_amd"))

from oracle import oracle  # noqa: E402
from openmini_qmm import synth  # noqa: E402


def main():
    out = {}
    for qtype, tag, (N, K) in ((2, "q4", (24, 128)), (7, "q8", (16, 96))):
        blocks = synth.weight_blocks(qtype, N, K, seed=0x5EED0000 + qtype)
        x = synth.normal(0x5EED8000 + qtype, (2, K), 1.0)
        out[f"{tag}_shape"] = np.array([N, K], dtype=np.int64)
        out[f"{tag}_blocks"] = blocks
        out[f"{tag}_x"] = x
        out[f"{tag}_w"] = oracle.dequantize(qtype, blocks, N * K)
        out[f"{tag}_y"] = oracle.linear_f64(qtype, blocks, N, K, x)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "oracle_small.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
