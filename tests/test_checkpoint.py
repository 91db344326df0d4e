"""Checkpoint files on the host (no GPU): the header, the text-group walk of
q3vl_checkpoint_text_layout, the writer and the RoPE tables, against the
reference's own loader init_model_weights (model/src/load_model.cpp:50-246)
and qwen_rope_precompute (:413-490) compiled into oracle/_ref; and the oracle's
restatement of the exporter's quantizer (export_bin/export_qwen_bin.py:260-275)
pinned by closed forms.

Bars: layout and RoPE tables bit-exact against the reference; quantizer
closed forms exact.
"""
import ctypes

import numpy as np
import pytest

from q3vl_int8 import checkpoint as ck

TINY = dict(vocab=64, hidden=64, intermediate=128, layers=2, heads=2, kv_heads=1,
            max_position=4096, rope_theta=10000, rms_eps=1e-6,
            vision_hidden=8, vision_depth=18, vision_patch=2, vision_spatial_merge=2,
            vision_temporal_patch=2, vision_heads=2, vision_intermediate=16, out_hidden=64,
            image_token_id=51, vision_start_token_id=52, vision_end_token_id=53,
            video_token_id=54, text_bits=8, group_size=32, vision_bits=32, group_quantized=1)
# vision_depth >= 18: the loader marks deep-stack layers 5, 11 and 17
# (load_model.cpp:108-111).

# Vision weights the loader transposes in memory after mapping them
# (Tensor::permute copies, utils/src/tensor.cpp:304; load_model.cpp:203-238).
PERMUTED = {"attn_proj_w": (0, 2, 1), "attn_qkv_w": (0, 1, 3, 2), "mlp1_w": (0, 2, 1),
            "mlp2_w": (0, 2, 1), "d_mlp1_w": (0, 2, 1), "d_mlp2_w": (0, 2, 1),
            "merge_mlp1_w": (1, 0), "merge_mlp2_w": (1, 0)}


def _tiny_text(hdr, orc, seed):
    rng = np.random.default_rng(seed)
    text, floats = {}, {}
    for n, shape in ck.text_shapes(hdr).items():
        x = rng.standard_normal(shape).astype(np.float32)
        floats[n] = x
        if hdr["text_bits"] == 8:
            text[n] = orc.quantize_groupwise(x, ck.quant_group(hdr, n))
        else:
            text[n] = x
    return text, floats


def _tiny_vision(hdr, seed):
    rng = np.random.default_rng(seed)
    return {n: rng.standard_normal(s).astype(np.float32)
            for n, s in ck.vision_shapes(hdr).items()}


def test_header_is_100_bytes_and_round_trips(tmp_path):
    b = ck.pack_header(TINY)
    assert len(b) == ck.HEADER_BYTES == ctypes.sizeof(ck.HeaderC)
    p = tmp_path / "h.bin"
    p.write_bytes(b)
    h = ck.read_header(str(p))
    for n, f in ck.HEADER_FIELDS:
        assert (np.float32(h[n]) == np.float32(TINY[n])) if f == "f" else h[n] == TINY[n], n


def test_short_file_is_an_error(tmp_path):
    import q3vl_int8
    p = tmp_path / "short.bin"
    p.write_bytes(b"\0" * 99)
    with pytest.raises(q3vl_int8.Q3VLError, match="shorter than the header"):
        ck.read_header(str(p))


@pytest.mark.parametrize("variant", [
    dict(),                                     # int8, group quantized
    dict(group_quantized=0),                    # int8, per-row scales except norms
    dict(text_bits=16, vision_bits=16),         # fp16 raw values
    dict(text_bits=32, group_size=64),          # fp32 raw values
])
def test_layout_matches_the_reference_loader(tmp_path, orc, ref, variant):
    hdr = dict(TINY, **variant)
    text, _ = _tiny_text(hdr, orc, 3)
    vision = _tiny_vision(hdr, 4)
    path = str(tmp_path / "tiny.bin")
    ck.write_checkpoint(path, hdr, text, vision)
    blob = open(path, "rb").read()

    fields, tensors, close = ref.checkpoint_open(path)
    try:
        for (n, f), v in zip(ck.HEADER_FIELDS, fields):
            assert (np.float32(v) == np.float32(hdr[n])) if f == "f" else v == hdr[n], n
        spans = ck.text_layout(hdr)
        elem = {8: 1, 16: 2, 32: 4}[hdr["text_bits"]]
        for i, n in enumerate(ck.TEXT_TENSORS):
            sp, t = spans[n], tensors[i]
            assert t["count"] == sp["data_count"], n
            nb = sp["data_count"] * elem
            assert ctypes.string_at(t["data"], nb) == blob[sp["data_offset"]:sp["data_offset"] + nb], n
            if hdr["text_bits"] == 8:
                assert t["group"] == sp["group"] == ck.quant_group(hdr, n), n
                sb = sp["scales_count"] * 4
                assert ctypes.string_at(t["scales"], sb) == \
                    blob[sp["scales_offset"]:sp["scales_offset"] + sb], n
            else:
                assert sp["scales_count"] == 0 and not t["scales"], n
        vdt = np.float32 if hdr["vision_bits"] == 32 else np.float16
        for j, n in enumerate(ck.VISION_TENSORS):
            t = tensors[len(ck.TEXT_TENSORS) + j]
            v = vision[n].transpose(PERMUTED[n]) if n in PERMUTED else vision[n]
            want = np.ascontiguousarray(v.astype(vdt)).tobytes()
            assert t["count"] * vdt().itemsize == len(want), n
            assert ctypes.string_at(t["data"], len(want)) == want, n
        # the file ends where the last vision group ends
        last = tensors[-1]
        end = spans["final_norm"]["data_offset"] + spans["final_norm"]["data_count"] * elem
        vbytes = sum(int(np.prod(s)) for s in ck.vision_shapes(hdr).values()) * vdt().itemsize
        assert len(blob) == end + vbytes and last["count"] == vision["merge_norm_w"].size
    finally:
        close()


def test_layout_rejects_a_partial_group():
    import q3vl_int8
    hdr = dict(TINY, group_size=48)  # 64-wide rows are not whole groups of 48
    with pytest.raises(q3vl_int8.Q3VLError, match="not whole groups"):
        ck.text_layout(hdr)


@pytest.mark.parametrize("theta,hidden,heads,rows", [
    (5000000, 2048, 16, 3072),  # the model's tables (load_model.cpp:93 fixes seq_len 3072)
    (10000, 512, 8, 300),
])
def test_rope_tables_match_the_reference(ref, theta, hidden, heads, rows):
    hd = hidden // heads
    cos, sin = ck.rope_tables(theta, hd, rows)
    rc, rs = ref.rope_precompute(theta, hidden, heads, rows)
    # plane 0 (T) is what text positions read; a text position's three
    # sections are equal, so every plane matches
    for p in range(3):
        np.testing.assert_array_equal(cos.view(np.uint32), rc[p].view(np.uint32))
        np.testing.assert_array_equal(sin.view(np.uint32), rs[p].view(np.uint32))


def test_rope_tables_closed_forms():
    cos, sin = ck.rope_tables(10000, 64, 50)
    assert (cos[0] == 1).all() and (sin[0] == 0).all()        # position 0
    p = np.arange(50, dtype=np.float64)
    # inv_freq[0] = 1: column 0 is cos(p), sin(p)
    np.testing.assert_allclose(cos[:, 0], np.cos(p), atol=2e-7)
    np.testing.assert_allclose(sin[:, 0], np.sin(p), atol=2e-7)
    # column i at 10000^(-2i/64), in double: within a few fp32 ulps of the argument
    inv = 10000.0 ** (-2.0 * np.arange(32) / 64)
    np.testing.assert_allclose(cos, np.cos(p[:, None] * inv[None]), atol=3e-6)
    np.testing.assert_allclose(cos ** 2 + sin ** 2, 1.0, atol=1e-6)


# ------------------------------------------------ the exporter's quantizer
def test_oracle_quantizer_exact_scales_and_values(orc):
    # group g holds k * (g + 1) with one element at 127 (g + 1): m >= 1 absorbs
    # the 1e-8, so s = 127 (g + 1) / 127 = g + 1 exactly and q = k
    rng = np.random.default_rng(5)
    for group in (32, 64, 128, 2048):
        ng = 24
        k = rng.integers(-127, 128, size=(ng, group))
        k[:, 0] = np.where(rng.random(ng) < 0.5, 127, -127)
        rng.permuted(k, axis=1, out=k)
        x = (k * (np.arange(ng)[:, None] + 1)).astype(np.float32)
        q, s = orc.quantize_groupwise(x, group)
        np.testing.assert_array_equal(s, np.arange(1, ng + 1, dtype=np.float32))
        np.testing.assert_array_equal(q.astype(np.int64), k)


def test_oracle_quantizer_zero_group_and_ties(orc):
    x = np.zeros(64, np.float32)
    # second group: max 127 -> s = 1; ties at n + 1/2 go to the even neighbour
    ties = [0.5, 1.5, 2.5, -2.5, -0.5, 125.5, 126.5, -126.5, 3.49999976]
    x[32:32 + len(ties)] = ties
    x[63] = 127.0
    q, s = orc.quantize_groupwise(x, 32)
    assert s[0] == np.float32(np.float32(1e-8) / np.float32(127))
    assert not q[:32].any()
    assert s[1] == 1.0
    assert list(q[32:32 + len(ties)]) == [0, 2, 2, -2, 0, 126, 126, -126, 3]
    assert q[63] == 127


def test_oracle_quantizer_error_bound(orc):
    rng = np.random.default_rng(6)
    x = (rng.standard_normal(64 * 300) * rng.uniform(1e-3, 10, 64 * 300)).astype(np.float32)
    q, s = orc.quantize_groupwise(x, 64)
    g = x.reshape(-1, 64).astype(np.float64)
    sd = s.astype(np.float64)[:, None]
    assert (np.abs(q.reshape(-1, 64) * sd - g) <= sd * (0.5 + 1e-6)).all()
    # the largest magnitude of each group lands on +-127
    am = np.abs(g).argmax(axis=1)
    np.testing.assert_array_equal(np.abs(q.reshape(-1, 64)[np.arange(300), am]), 127)
    np.testing.assert_array_equal(np.sign(q.reshape(-1, 64)[np.arange(300), am]),
                                  np.sign(g[np.arange(300), am]))


def test_writer_rejects_wrong_shapes(tmp_path, orc):
    hdr = dict(TINY)
    text, _ = _tiny_text(hdr, orc, 8)
    q, sc = text["k"]
    bad = dict(text, k=(q[:, :-1], sc))  # one row short
    with pytest.raises(ValueError, match="k:"):
        ck.write_checkpoint(str(tmp_path / "bad.bin"), hdr, bad)
    bad = dict(text, k=(q, sc[:-1]))     # one scale short
    with pytest.raises(ValueError, match="k:"):
        ck.write_checkpoint(str(tmp_path / "bad2.bin"), hdr, bad)
    vis = {"pos_emb_w": np.zeros((10, 8), np.float32)}
    with pytest.raises(ValueError, match="pos_emb_w"):
        ck.write_checkpoint(str(tmp_path / "bad3.bin"), hdr, text, vis)


def test_raw_text_export_needs_no_device(tmp_path, orc):
    """fp32 text weights are written as they are (no quantizer involved)."""
    hdr = dict(TINY, text_bits=32)
    _, floats = _tiny_text(hdr, orc, 9)
    a, b = str(tmp_path / "a.bin"), str(tmp_path / "b.bin")
    ck.export_checkpoint(a, hdr, floats)
    ck.write_checkpoint(b, hdr, floats)
    assert open(a, "rb").read() == open(b, "rb").read()
