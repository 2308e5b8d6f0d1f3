"""Loaders for the committed golden fixtures (written by tests/golden/make_golden.py)."""

import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name: str):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def qmm_cases():
    z = load("qmm_small.npz")
    out = []
    for ci, (m, k, n) in enumerate(z["shapes"]):
        out.append(dict(m=int(m), k=int(k), n=int(n), **{f: z[f"c{ci}_{f}"] for f in ("x", "w", "s", "b", "deq", "exact", "y")}))
    return out


def dequant_table_weights():
    """The fixture's (s, b) pairs as a weight matrix: row i = pair i, K = 64 (one group) holding
    the codes 0..15 four times; expected[i, k] = fixture expected[i, k % 16]."""
    z = load("dequant_table.npz")
    n = z["scales"].shape[0]
    codes = np.tile(np.arange(16, dtype=np.uint32), 4)  # k -> code k % 16
    words = np.zeros(8, dtype=np.uint32)
    for c in range(8):
        for i in range(8):
            words[c] |= codes[8 * c + i] << np.uint32(4 * i)
    w = np.tile(words, (n, 1))
    expected = np.tile(z["expected"], (1, 4))
    return w, z["scales"].reshape(n, 1), z["biases"].reshape(n, 1), expected, np.tile(z["single_rounding"], (1, 4))
