"""Deterministic synthetic inputs shared by the golden-vector writer, the tests
and bench.py (numpy PCG64; shapes and distributions of the BASELINE configs):
W int8 uniform on [-127, 127], S fp32 U(0.001, 0.02) per group, A fp32 N(0,1).
"""
from __future__ import annotations

import hashlib

import numpy as np


def make_case(seed: int, M: int, N: int, K: int, gs: int):
    rng = np.random.default_rng(seed)
    A = rng.standard_normal((M, K), dtype=np.float32)
    W = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    S = rng.uniform(0.001, 0.02, size=(N, K // gs)).astype(np.float32)
    return A, W, S


def sha256(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def tie_group_row(orc, gs: int = 64, K: int = 1024):
    """An activation row whose first group quantizes with a_s == 1.0 exactly,
    so that q = round-half-even(x) on half-integer inputs (0.5 -> 0, 1.5 -> 2,
    2.5 -> 2, ...). Found by search with the oracle; deterministic."""
    ties = np.array([0.5, 1.5, 2.5, 3.5, -0.5, -1.5, -2.5, -3.5], np.float32)
    rng = np.random.default_rng(1234)
    for _ in range(20000):
        small = rng.choice(ties, size=gs - 1)
        rest = 1032256.0 - float(np.sum(small.astype(np.float64) ** 2))
        for delta in range(-40, 41):
            big = np.float32(np.sqrt(rest) + delta * 2e-6)
            row = np.zeros((1, K), np.float32)
            row[0, 0] = big
            row[0, 1:gs] = small
            row[0, gs:] = rng.standard_normal(K - gs).astype(np.float32)
            q, s = orc.quantize_rows(row, gs)
            if s[0, 0] == np.float32(1.0):
                return row
    raise RuntimeError("no tie row found")
