"""Writes tests/golden/golden_int8.npz from the reference's own compiled code.

Run in the development container (needs oracle/_ref/libref_q3vl.so, built by
`make -C oracle ref` from /root/reference). Inputs are regenerated from seeds
by tests/golden/gen.py; the fixture stores their SHA-256 so a generator drift
fails loudly instead of comparing against the wrong inputs. Outputs stored:
  lin_<name>_C     reference linear() output for a seeded case
  probe_<name>_C   reference linear() on the one-hot probe (W = identity rows,
                   S = 1): C[m, k] = fl(q[m,k] * a_s[m, k/gs]) exactly, which
                   pins the quantizer through the reference's observable output
  swiglu_out       reference swiglu() on seeded / special values
  tie_C            reference linear() probe on the round-half-even tie row
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, HERE)

from checkers import Oracle, Reference  # noqa: E402
from gen import make_case, sha256, tie_group_row  # noqa: E402

# (name, seed, M, N, K, gs): lane path (M=1, N>=1024, K>=1024) and general path.
LIN_CASES = [
    ("lane_1k_gs64", 11, 1, 1024, 1024, 64),
    ("lane_2k_gs64", 12, 1, 2048, 2048, 64),
    ("lane_gs32", 13, 1, 1024, 1024, 32),
    ("lane_gs128", 14, 1, 1024, 2048, 128),
    ("lane_gs16", 15, 1, 1024, 1024, 16),
    ("lane_k6144", 16, 1, 1024, 6144, 64),
    ("lane_tail_n1028", 17, 1, 1028, 1024, 64),
    ("gen_m1_n512", 21, 1, 512, 2048, 64),
    ("gen_m2", 22, 2, 256, 512, 64),
    ("gen_m8", 23, 8, 1000, 2048, 64),
    ("gen_m5_gs32", 24, 5, 1028, 1024, 32),
    ("gen_m3_gs128", 25, 3, 128, 1024, 128),
    ("gen_m16", 26, 16, 384, 1024, 64),
    ("gen_m1_k512", 27, 1, 2048, 512, 64),
]
PROBE_CASES = [("lane", 31, 1, 1024, 64), ("general", 32, 2, 1024, 64)]


def probe_inputs(seed, M, K, gs):
    rng = np.random.default_rng(seed)
    A = rng.standard_normal((M, K), dtype=np.float32) * np.float32(3.0)
    W = np.eye(K, dtype=np.int8)
    S = np.ones((K, K // gs), np.float32)
    return A, W, S


def swiglu_inputs():
    rng = np.random.default_rng(41)
    g = (rng.standard_normal(4096) * 4).astype(np.float32)
    u = rng.standard_normal(4096).astype(np.float32)
    special = np.array([0.0, -0.0, 1e-30, -1e-30, 20.0, -20.0, 88.0, -88.0, 90.0, -90.0,
                        1e-8, -1e-8, 0.5, -0.5, 3.0, -3.0], np.float32)
    g[: special.size] = special
    return g, u


def main():
    ref = Reference.load()
    if ref is None:
        raise SystemExit("oracle/_ref/libref_q3vl.so missing: run `make -C oracle ref`")
    orc = Oracle.load()
    out, meta = {}, {"lin": [], "probe": []}
    for name, seed, M, N, K, gs in LIN_CASES:
        A, W, S = make_case(seed, M, N, K, gs)
        out[f"lin_{name}_C"] = ref.linear(A, W, S, gs)
        meta["lin"].append(dict(name=name, seed=seed, M=M, N=N, K=K, gs=gs, sha256=sha256(A, W, S)))
    for name, seed, M, K, gs in PROBE_CASES:
        A, W, S = probe_inputs(seed, M, K, gs)
        out[f"probe_{name}_A"] = A
        out[f"probe_{name}_C"] = ref.linear(A, W, S, gs)
        meta["probe"].append(dict(name=name, seed=seed, M=M, K=K, gs=gs))
    row = tie_group_row(orc)
    out["tie_A"] = row
    W = np.eye(row.shape[1], dtype=np.int8)
    out["tie_C"] = ref.linear(row, W, np.ones((row.shape[1], row.shape[1] // 64), np.float32), 64)
    g, u = swiglu_inputs()
    out["swiglu_gate"], out["swiglu_up"] = g, u
    out["swiglu_out"] = ref.swiglu(g, u)
    np.savez_compressed(os.path.join(HERE, "golden_int8.npz"), **out)
    with open(os.path.join(HERE, "golden_int8.json"), "w") as f:
        json.dump(meta, f, indent=1)
    print("wrote", sum(v.nbytes for v in out.values()), "bytes of vectors")


if __name__ == "__main__":
    main()
