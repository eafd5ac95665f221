"""Writes tests/golden/oracle/IQ3_S.{raw,f32}: 16 IQ3_S blocks (random bytes, f16 d in [0.01, 0.02), the design of the
reference's random_tensor, tests/kernels.rs:1473-1550) and their dequantization by the C oracle.

These vectors are ORACLE-DERIVED, NOT REFERENCE-HELD: the reference holds no IQ3_S vector, and its Rust dequant
(src/quant/mod.rs:345-361) cannot be run here. They pin the oracle and the GPU kernel against later changes; the
oracle's IQ3_S arithmetic itself is pinned by the known-answer block and the dot/dequant cross-check in
tests/test_oracle.py. Run from the repo root: python -m tests.golden.make_oracle_vectors
"""
import os

import numpy as np

from oracle import oracle as O
from rustingstrata_amd import ggml
from tests.helpers import random_blocks

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "oracle")


def main():
    os.makedirs(OUT, exist_ok=True)
    raw = random_blocks(ggml.IQ3_S, 1, 16 * 256, seed=3210).reshape(-1)
    y = O.dequant(ggml.IQ3_S, raw, 16 * 256)
    raw.tofile(os.path.join(OUT, "IQ3_S.raw"))
    y.astype(np.float32).tofile(os.path.join(OUT, "IQ3_S.f32"))
    print(f"wrote {raw.size} bytes, {y.size} floats to {OUT}")


if __name__ == "__main__":
    main()
