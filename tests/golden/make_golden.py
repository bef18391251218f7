"""Writes tests/golden/oracle_vectors.npz: seeded synthetic GGUF blocks, an
activation row, and the oracle's dequantized values and reference-path
matmul outputs, frozen once the oracle was pinned by tests/test_oracle.py.

The reference (Rust) cannot be built or run here, so these vectors come from
the oracle; they guard the oracle against unintended changes.
Run: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402
from tests._util import synth_blocks  # noqa: E402


def main():
    rng = np.random.default_rng(0x60D)
    out = {"a": rng.standard_normal(1024).astype(np.float32)}
    for dt, name, n, k in ((O.Q8_0, "q8_0", 24, 1024), (O.Q4_K, "q4_k", 24, 1024), (O.Q6_K, "q6_k", 24, 1024)):
        be = O.BLOCK_ELEMS[dt]
        raw = synth_blocks(dt, n * (k // be), 0x60D + dt)
        out[name + "_raw"] = raw
        out[name + "_shape"] = np.array([n, k])
        out[name + "_deq"] = O.dequant(dt, raw, n * k)
        out[name + "_mm"] = O.reference_matmul(dt, out["a"][:k], raw, 1, n, k)
    np.savez_compressed(os.path.join(os.path.dirname(os.path.abspath(__file__)), "oracle_vectors.npz"), **out)


if __name__ == "__main__":
    main()
