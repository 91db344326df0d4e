"""Pins the oracle's chunked attention order (orc_attention_chunked, the
GPU's Q3VL_ATTN_CHUNKED; no counterpart in the reference, whose softmax and
value sum run over all positions in one order) by what the mathematics
fixes. It is softmax(q k / sqrt(d)) v computed with the reference's exp256
polynomial, whose relative error (about 2e-4 here) bounds both orders:
the chunked and the reference-order oracles each stay within 5e-4 (relative
to the output scale) of a float64 brute force, and within 5e-4 of each
other (measured: up to 3.1e-4). Equal scores give the plain mean of the value rows; a score 40 above
the rest selects that value row exactly; a single chunk (at most 64
positions) is its e-weighted values over its own sum. A score more than
88.38 below the maximum makes exp256 return -inf (2^-128 is built as -inf),
which zeroes the head in the reference order (text_layer.cpp:512-515): the
chunked order gives zeros there too, also when no chunk spans that gap by
itself (a chunk at -50 and -100 against a maximum of 0 elsewhere: each factor
exp256(-50) is finite, the reference's exp256(-100) is not), through each
chunk's smallest finite score. A dropped chunk, a wrong chunk weight or a
value row off by one position fails these.
"""
import numpy as np
import pytest

H, KV, D = 4, 2, 128


def brute(q, kc, vc, pos):
    """float64 softmax attention over positions 0..pos."""
    kvm = H // KV
    out = np.zeros((H, D))
    for h in range(H):
        k = kc[h // kvm, :pos + 1].astype(np.float64)
        v = vc[h // kvm, :pos + 1].astype(np.float64)
        s = k @ q[h * D:(h + 1) * D].astype(np.float64) / np.sqrt(D)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ v
    return out.reshape(-1)


def case(seed, S, qscale=1.0):
    rng = np.random.default_rng(seed)
    q = (rng.standard_normal(H * D) * qscale).astype(np.float32)
    kc = rng.standard_normal((KV, S, D)).astype(np.float16).astype(np.float32)
    vc = rng.standard_normal((KV, S, D)).astype(np.float16).astype(np.float32)
    return q, kc, vc


@pytest.mark.parametrize("pos", [0, 1, 63, 64, 65, 127, 128, 300, 700, 1023])
def test_chunked_matches_brute_force_and_reference_order(orc, pos):
    S = 1024
    for seed, qs in ((pos + 11, 1.0), (pos + 12, 3.0)):
        q, kc, vc = case(seed, S, qs)
        got = orc.attention_chunked(q, kc, vc, H, KV, D, S, pos)
        ref = orc.attention(q, kc, vc, H, KV, D, S, pos)
        bf = brute(q, kc, vc, pos)
        scale = np.abs(bf).max()
        assert np.abs(got - bf).max() <= 5e-4 * scale
        assert np.abs(ref - bf).max() <= 5e-4 * scale
        assert np.abs(got - ref).max() <= 5e-4 * scale
        if pos == 0:  # one position: both orders return that value row exactly
            np.testing.assert_array_equal(got, ref)


def test_equal_scores_give_the_mean(orc):
    S, pos = 256, 200
    _, kc, vc = case(5, S)
    q = np.zeros(H * D, np.float32)  # every score is 0: every e is exp256(0) = 1
    got = orc.attention_chunked(q, kc, vc, H, KV, D, S, pos).reshape(H, D)
    for h in range(H):
        mean = vc[h // (H // KV), :pos + 1].astype(np.float64).mean(axis=0)
        np.testing.assert_allclose(got[h], mean, rtol=0, atol=2e-6 * np.abs(mean).max())


def test_dominant_score_selects_its_row(orc):
    S, pos, hot = 512, 400, 137
    q, kc, vc = case(6, S)
    q[:] = 0.0
    q[::D] = 1.0  # component 0 of every head
    kc[:, :, 0] = -1.0
    kc[:, hot, 0] = 40.0 * np.sqrt(D)  # score 40, the rest -0.09
    got = orc.attention_chunked(q, kc, vc, H, KV, D, S, pos).reshape(H, D)
    for h in range(H):
        np.testing.assert_array_equal(got[h], vc[h // (H // KV), hot])


@pytest.mark.parametrize("pos", [0, 9, 63])
def test_single_chunk_is_its_own_fold(orc, pos):
    """One chunk: w_0 = exp256(0) = 1, so out = o_0 * (1 / l_0): the
    e-weighted values over the e sum (float64 here, exp256's error apart)."""
    S = 128
    q, kc, vc = case(pos + 3, S)
    got = orc.attention_chunked(q, kc, vc, H, KV, D, S, pos)
    kvm = H // KV
    for h in range(H):
        k = kc[h // kvm, :pos + 1].astype(np.float64)
        v = vc[h // kvm, :pos + 1].astype(np.float64)
        s = k @ q[h * D:(h + 1) * D].astype(np.float64) / np.sqrt(D)
        e = np.exp(s - s.max())
        want = (e @ v) / e.sum()
        np.testing.assert_allclose(got[h * D:(h + 1) * D], want, rtol=0,
                                   atol=5e-4 * np.abs(want).max())


@pytest.mark.parametrize("gap_chunk", [False, True])
def test_score_gap_past_exp256_range_zeroes_the_head(orc, gap_chunk):
    """One score 100 above the others: exp256(-100) is -inf, the sum is not
    positive, and the reference order writes zeros; the chunked order too,
    whether the low scores share the high score's chunk or fill another."""
    S, pos = 256, 150
    q, kc, vc = case(9, S)
    q[:] = 0.0
    q[::D] = 1.0
    kc[:, :, 0] = 0.0
    hot = 3 if gap_chunk else 100
    kc[:, hot, 0] = 100.0 * np.sqrt(D)
    if gap_chunk:  # positions 64.. hold the low scores, in their own chunks
        kc[:, :64, 0] = 100.0 * np.sqrt(D)
    for f in (orc.attention, orc.attention_chunked):
        got = f(q, kc, vc, H, KV, D, S, pos)
        np.testing.assert_array_equal(got, np.zeros_like(got))


def scored(S, scores):
    """q, k with score s_t = scores[t] for every head (dim 0 only)."""
    q, kc, vc = case(11, S)
    q[:] = 0.0
    q[::D] = 1.0
    kc[:, :, 0] = 0.0
    kc[:, :len(scores), 0] = np.asarray(scores, np.float64) * np.sqrt(D)
    return q, kc, vc


@pytest.mark.parametrize("low,zero", [(-100.0, True), (-80.0, False)])
def test_gap_spread_over_chunks(orc, low, zero):
    """Chunk 1 (positions 64..127) has its maximum at -50 and its other
    scores at `low`; chunks 0 and 2 are at 0, so M = 0. Within chunk 1 the
    spread is 50 or 30 and against M the chunk factor is exp256(-50): all
    finite. The reference order takes exp256(low - 0): -inf for -100 (the
    head is zeroed), finite for -80 (the orders agree to exp256's error)."""
    S, pos = 256, 150
    s = np.zeros(pos + 1)
    s[64:128] = low
    s[90] = -50.0
    q, kc, vc = scored(S, s)
    ref = orc.attention(q, kc, vc, H, KV, D, S, pos)
    got = orc.attention_chunked(q, kc, vc, H, KV, D, S, pos)
    if zero:
        np.testing.assert_array_equal(ref, np.zeros_like(ref))
        np.testing.assert_array_equal(got, np.zeros_like(got))
    else:
        assert np.abs(ref).max() > 0.01
        np.testing.assert_allclose(got, ref, rtol=0, atol=5e-4 * np.abs(ref).max())


def test_all_scores_minus_infinity_gives_zeros(orc):
    S, pos = 128, 70
    q, kc, vc = case(8, S)
    q[:] = 0.0
    q[::D] = 1.0
    kc[:, :, 0] = -np.inf  # every score -inf: no chunk has a finite max
    got = orc.attention_chunked(q, kc, vc, H, KV, D, S, pos)
    np.testing.assert_array_equal(got, np.zeros_like(got))
