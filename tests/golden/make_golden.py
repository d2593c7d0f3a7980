"""Writes tests/golden/golden.npz: seeded inputs and the oracle's bytes for
small shapes (regression fixtures for the PRNG and the quantizers).

Run from the repo root: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402
from smith_amd import prng  # noqa: E402

w_q4s = prng.randn((70, 24), 3, std=0.02)
w_q8 = prng.randn((64, 16), 4, std=0.02)
w_q4_0 = prng.randn((8, 64), 5, std=0.02)
np.savez_compressed(
    os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.npz"),
    splitmix_seed0=prng.splitmix64(0, 0, 8),
    randn_seed0=prng.randn((16,), 0),
    w_q4s=w_q4s, q4s_bytes=O.quantize_q4s(w_q4s),
    w_q8=w_q8, q8_bytes=O.quantize_q8(w_q8),
    w_q4_0=w_q4_0, q4_0_bytes=O.quantize_rows(O.GGML_Q4_0, w_q4_0),
)
print("wrote golden.npz")
