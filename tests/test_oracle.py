"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

1. Golden vectors written by the reference's own compiled code
   (tests/golden/make_golden.py): bit-exact.
2. One-hot probes: the reference's linear() with W = identity and S = 1 exposes
   fl(q * a_s) for every activation element; the oracle's (q, a_s) must give
   the same products bit for bit.
3. Known answers fixed by the mathematics of the quantizer: constant group ->
   +-127, single spike -> +-1016, zero group -> q = 0 and a_s = sqrt(1e-6)/127,
   exact half-integers under a_s == 1 -> round half to even.
4. Brute force: int64 group sums, |q - a/s| <= 1/2, a_s ~ rms/127 in float64.
5. A planted mistake (uncontracted general-path epilogue) must fail (1).
6. greedy_decode semantics: ties -> lowest index, NaN never wins, -inf/-FLT_MAX
   rows -> 0.
"""
import json
import os

import numpy as np
import pytest

from golden.gen import make_case, sha256
from golden.make_golden import LIN_CASES, probe_inputs, swiglu_inputs

GOLD = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def gold():
    return np.load(os.path.join(GOLD, "golden_int8.npz"))


@pytest.fixture(scope="module")
def meta():
    with open(os.path.join(GOLD, "golden_int8.json")) as f:
        return json.load(f)


@pytest.mark.parametrize("case", LIN_CASES, ids=[c[0] for c in LIN_CASES])
def test_oracle_matches_reference_golden(orc, gold, meta, case):
    name, seed, M, N, K, gs = case
    A, W, S = make_case(seed, M, N, K, gs)
    rec = [m for m in meta["lin"] if m["name"] == name][0]
    assert rec["sha256"] == sha256(A, W, S), "input generator drifted from the fixture"
    C = orc.linear(A, W, S, gs)
    np.testing.assert_array_equal(C.view(np.uint32), gold[f"lin_{name}_C"].view(np.uint32))


def test_planted_uncontracted_epilogue_fails(orc, gold):
    """The general path must fuse acc += (G*a_s)*w_s; three roundings differ."""
    name, seed, M, N, K, gs = [c for c in LIN_CASES if c[0] == "gen_m8"][0]
    A, W, S = make_case(seed, M, N, K, gs)
    C = orc.linear(A, W, S, gs, path="general_nofma")
    assert (C != gold[f"lin_{name}_C"]).mean() > 0.1


def test_planted_lane_order_fails(orc, gold):
    """The lane chain is not the general chain: swapping them must be caught."""
    name, seed, M, N, K, gs = [c for c in LIN_CASES if c[0] == "lane_2k_gs64"][0]
    A, W, S = make_case(seed, M, N, K, gs)
    C = orc.linear(A, W, S, gs, path="general")
    assert (C != gold[f"lin_{name}_C"]).mean() > 0.1


@pytest.mark.parametrize("name,M", [("lane", 1), ("general", 2)])
def test_quantizer_pinned_by_one_hot_probe(orc, gold, name, M):
    A = gold[f"probe_{name}_A"]
    K = A.shape[1]
    q, a_s = orc.quantize_rows(A, 64)
    prod = (q.astype(np.float32) * np.repeat(a_s, 64, axis=1)).astype(np.float32)
    np.testing.assert_array_equal(prod.view(np.uint32), gold[f"probe_{name}_C"].view(np.uint32))
    # and the full oracle linear on the probe matches too
    _, W, S = probe_inputs(0, M, K, 64)
    C = orc.linear(A, W, S, 64)
    np.testing.assert_array_equal(C.view(np.uint32), gold[f"probe_{name}_C"].view(np.uint32))


def test_round_half_even_ties(orc, gold):
    row = gold["tie_A"]
    q, a_s = orc.quantize_rows(row, 64)
    assert a_s[0, 0] == np.float32(1.0)
    x = row[0, 1:64].astype(np.float64)
    assert np.all(np.abs(x - np.trunc(x)) == 0.5)  # all exact ties
    np.testing.assert_array_equal(q[0, 1:64], np.round(x).astype(np.int16))  # numpy: half-even
    assert np.any(np.round(x) != np.trunc(x + np.sign(x) * 0.5))  # half-away would differ
    prod = (q.astype(np.float32) * np.repeat(a_s, 64, axis=1)).astype(np.float32)
    np.testing.assert_array_equal(prod.view(np.uint32), gold["tie_C"].view(np.uint32))


def test_quantizer_known_answers(orc):
    K, gs = 256, 64
    A = np.zeros((1, K), np.float32)
    A[0, 0:64] = 0.75            # constant group
    A[0, 64 + 17] = -5.0         # single spike
    # group 2 all zero
    A[0, 192:256] = -2.0         # constant negative group
    q, s = orc.quantize_rows(A, gs)
    assert np.all(q[0, 0:64] == 127)
    assert q[0, 64 + 17] == -1016 and np.count_nonzero(q[0, 64:128]) == 1
    assert np.all(q[0, 128:192] == 0)
    assert s[0, 2] == np.float32(np.sqrt(np.float32(1e-6))) * np.float32(1.0 / 127.0)
    assert np.all(q[0, 192:256] == -127)


def test_quantizer_brute_force(orc):
    rng = np.random.default_rng(5)
    for gs in (16, 32, 64, 128, 256):
        A = (rng.standard_normal((4, 1024)) * rng.uniform(0.01, 100, (4, 1))).astype(np.float32)
        q, s = orc.quantize_rows(A, gs)
        a = A.astype(np.float64).reshape(4, -1, gs)
        rms = np.sqrt((a ** 2).mean(-1) + 1e-6)
        np.testing.assert_allclose(s, rms / 127.0, rtol=2e-6)
        inv = (np.float32(1.0) / s).astype(np.float32)
        p = (A.reshape(4, -1, gs) * inv[..., None]).astype(np.float32)
        assert np.all(np.abs(q.reshape(4, -1, gs) - p.astype(np.float64)) <= 0.5)
        assert np.abs(q).max() <= 1016


def test_group_sums_brute_force(orc):
    for (M, N, K, gs) in [(1, 1024, 1024, 64), (3, 64, 512, 32), (2, 1024, 2048, 128)]:
        A, W, S = make_case(7, M, N, K, gs)
        C, G = orc.linear(A, W, S, gs, groups=True)
        q, _ = orc.quantize_rows(A, gs)
        ref = np.einsum("mgk,ngk->mng", q.reshape(M, -1, gs).astype(np.int64),
                        W.reshape(N, -1, gs).astype(np.int64))
        np.testing.assert_array_equal(G.astype(np.int64), ref)


def test_dispatch_rule(orc):
    assert orc.uses_lane_path(1, 1024, 1024)
    assert not orc.uses_lane_path(1, 1023, 4096)
    assert not orc.uses_lane_path(1, 4096, 512)
    assert not orc.uses_lane_path(2, 4096, 4096)


def test_swiglu_matches_reference_golden(orc, gold):
    g, u = swiglu_inputs()
    np.testing.assert_array_equal(g, gold["swiglu_gate"])
    out = orc.swiglu(g, u)
    np.testing.assert_array_equal(out.view(np.uint32), gold["swiglu_out"].view(np.uint32))


def _greedy(x):
    best, idx = -np.finfo(np.float32).max, 0
    for i, v in enumerate(x):
        if v > best:
            best, idx = v, i
    return idx


def test_argmax_semantics(orc):
    fmax = np.finfo(np.float32).max
    cases = [
        np.array([1, 3, 3, 2], np.float32),                      # tie -> first
        np.array([np.nan, 1, np.nan, 1], np.float32),            # NaN never wins
        np.array([-np.inf, -np.inf], np.float32),                # nothing > -FLT_MAX -> 0
        np.array([-fmax, -fmax, -1e30], np.float32),             # -FLT_MAX not selected
        np.array([-0.0, 0.0, -0.0], np.float32),                 # +-0 equal -> first
        np.array([np.nan, np.nan], np.float32),
    ]
    rng = np.random.default_rng(3)
    for _ in range(20):
        x = rng.integers(-5, 5, 200).astype(np.float32)
        cases.append(x)
    for x in cases:
        assert orc.argmax_rows(x)[0] == _greedy(x)
    assert orc.argmax_rows(cases[0])[0] == 1
    assert orc.argmax_rows(cases[1])[0] == 1
    assert orc.argmax_rows(cases[2])[0] == 0


def test_oracle_matches_compiled_reference_live(orc, ref):
    """Where oracle/_ref is built (development container): more random shapes."""
    rng = np.random.default_rng(9)
    for (M, N, K, gs) in [(1, 1024, 1024, 64), (1, 70000, 1024, 64), (4, 512, 1024, 64),
                          (12, 64, 2048, 128), (1, 2048, 3072, 32)]:
        A = rng.standard_normal((M, K)).astype(np.float32)
        W = rng.integers(-127, 128, (N, K)).astype(np.int8)
        S = rng.uniform(0.001, 0.02, (N, K // gs)).astype(np.float32)
        np.testing.assert_array_equal(orc.linear(A, W, S, gs).view(np.uint32),
                                      ref.linear(A, W, S, gs).view(np.uint32))
