"""Pins the oracle's decode step (oracle/decode_oracle.c, a restatement of
model/src/forward.cpp:458-720) against the reference's own compiled code.

Per op: the two RMS norms (whose sum of squares the reference leaves to the
compiler's `omp simd reduction`: 8 FMA lanes folded left to right), RoPE,
softmax and the attention of one layer are compared bit for bit with the
compiled reference. End to end: whole decode steps of a small synthetic int8
model through the reference's forward_text (fp32 KV cache, as the reference)
against the oracle in its fp32-cache mode: greedy ids equal, logits within
the tolerance written below.
"""
import numpy as np
import pytest

from golden.gen import SMALL, make_kv_cache, make_text_model, quantize_groupwise, rope_tables


def norm_weights(n, gs, seed):
    rng = np.random.default_rng(seed)
    return quantize_groupwise(rng.uniform(0.9, 1.1, n).astype(np.float32), gs)


@pytest.mark.parametrize("n", [128, 2048])
def test_rms_norms_vs_reference(orc, ref, n):
    rng = np.random.default_rng(n)
    w, ws = norm_weights(n, 64, 3)
    for scale in (1e-3, 1.0, 300.0, 1e-2, 7.0, 1e3):
        x = (rng.standard_normal(n) * scale).astype(np.float32)
        a, b = orc.rms_norm_i8(x, w, ws, 64, 1e-6), ref.rms_norm_i8(x, w, ws, 64, 1e-6)
        np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
        xb = np.tile(x[:128], 16) if n == 128 else x
        bt = 16 if n == 128 else 1
        a = orc.rms_norm_inplace_i8(xb, w[:xb.size // bt], ws, 64, 1e-6, bt)
        b = ref.rms_norm_inplace_i8(xb, w[:xb.size // bt], ws, 64, 1e-6, bt)
        np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


def test_rope_vs_reference(orc, ref):
    cos_t, sin_t = rope_tables(3072, 128, 5e6)
    x = np.random.default_rng(1).standard_normal(16 * 128).astype(np.float32)
    for pos in (0, 1, 1024, 3071):
        np.testing.assert_array_equal(orc.rope(x, cos_t[pos], sin_t[pos], 16, 128),
                                      ref.rope(x, cos_t, sin_t, 16, 128, pos))


def test_exp_polynomial_and_softmax_vs_reference(orc, ref):
    rng = np.random.default_rng(2)
    for n in (1, 7, 8, 9, 64, 1025, 3000):
        x = (rng.standard_normal(n) * 4).astype(np.float32)
        if n > 8:
            x[3] = -np.inf
        np.testing.assert_array_equal(orc.softmax(x), ref.softmax(x))
    # every score is -inf -> zeros (text_layer.cpp:466-469)
    x = np.full(9, -np.inf, np.float32)
    np.testing.assert_array_equal(orc.softmax(x), np.zeros(9, np.float32))


@pytest.mark.parametrize("pos", [0, 5, 63, 64, 1024])
def test_attention_vs_reference(orc, ref, pos):
    rng = np.random.default_rng(pos)
    H, KV, D, S = 16, 8, 128, 1100
    q = rng.standard_normal(H * D).astype(np.float32)
    kc = rng.standard_normal((KV, S, D)).astype(np.float16).astype(np.float32)
    vc = rng.standard_normal((KV, S, D)).astype(np.float16).astype(np.float32)
    a = orc.attention(q, kc, vc, H, KV, D, S, pos)
    b = ref.attention(q, kc, vc, H, KV, D, S, pos)
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


def test_fp16_conversions(orc):
    import ctypes
    L = orc.lib
    L.orc_float_to_half.restype = ctypes.c_uint16
    L.orc_float_to_half.argtypes = [ctypes.c_float]
    L.orc_half_to_float.restype = ctypes.c_float
    L.orc_half_to_float.argtypes = [ctypes.c_uint16]
    rng = np.random.default_rng(4)
    xs = np.concatenate([rng.standard_normal(3000) * 10 ** rng.uniform(-8, 5, 3000),
                         [0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e-8, 6e-8, 3e-8, np.inf, -np.inf]])
    xs = xs.astype(np.float32)
    want = xs.astype(np.float16).view(np.uint16)
    got = np.array([L.orc_float_to_half(float(v)) for v in xs], np.uint16)
    np.testing.assert_array_equal(got, want)
    hs = np.arange(0, 65536, 7, dtype=np.uint16)
    hs = hs[(hs & 0x7C00) != 0x7C00]
    back = np.array([L.orc_half_to_float(int(h)) for h in hs], np.float32)
    np.testing.assert_array_equal(back, hs.view(np.float16).astype(np.float32))


@pytest.mark.parametrize("gs", [64, 32, 128])  # the exporter's group sizes (export_qwen_bin.py:371)
def test_decode_steps_vs_reference_forward_text(orc, ref, gs):
    """Four chained decode steps of a small model: the reference's
    forward_text (fp32 caches) vs the oracle in fp32-cache mode. Logits, the
    cache rows each step writes and the greedy ids are all bit-exact."""
    dims = dict(SMALL, gs=gs)
    m = make_text_model(11, dims)
    k16, v16 = make_kv_cache(12, dims, ctx=100)
    kr, vr = k16.astype(np.float32), v16.astype(np.float32)
    ko, vo = kr.copy(), vr.copy()
    dec = ref.decoder(dims, m, kr, vr)
    token = 7
    try:
        for step in range(4):
            pos = 100 + step
            lr = dec.step(token, pos)
            nid, lo = orc.decode_step(dims, m, ko, vo, token, pos, kv_fp16=False)
            np.testing.assert_array_equal(lo.view(np.uint32), lr.view(np.uint32))
            np.testing.assert_array_equal(ko.view(np.uint32), kr.view(np.uint32))
            np.testing.assert_array_equal(vo.view(np.uint32), vr.view(np.uint32))
            assert nid == int(np.argmax(lr)), (step, nid, int(np.argmax(lr)))
            token = nid
    finally:
        dec.close()
