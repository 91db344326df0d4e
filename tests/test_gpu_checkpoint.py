"""Checkpoint files on the GPU: the exporter's quantizer
(q3vl_quantize_groupwise, export_bin/export_qwen_bin.py:260-275) against the
oracle's restatement, the device-quantized export against the oracle-quantized
file, and q3vl_checkpoint_load (model/src/load_model.cpp:50-246 to device
residency) followed by decode steps against the oracle.

Bars: int8 values, fp32 scales, file bytes, device bytes, logits, caches and
greedy ids bit-exact.
"""
import ctypes

import numpy as np
import pytest

from golden.gen import SMALL, make_kv_cache, make_text_model

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()
    import q3vl_int8
    from q3vl_int8 import checkpoint as ck
    # the HIP runtime torch and the library already share (same soname)
    hip = ctypes.CDLL("libamdhip64.so.7")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    hip.hipMemcpy.restype = ctypes.c_int
    return torch, q3vl_int8, ck, hip


def _d2h(hip, ptr, nbytes, dtype):
    out = np.empty(nbytes // np.dtype(dtype).itemsize, dtype)
    assert hip.hipMemcpy(out.ctypes.data, ptr, nbytes, 2) == 0  # hipMemcpyDeviceToHost
    return out


def _quantize(dev, x, group):
    torch, q3, _, _ = dev
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    q, s = q3.quantize_groupwise(xd, group)
    torch.cuda.synchronize()
    return q.cpu().numpy(), s.cpu().numpy()


# group sizes of every kernel: float4 lanes (4..256, powers of two), a wave
# per group (multiples of 4 above 256), one value per lane (the rest)
@pytest.mark.parametrize("group,ngroups", [(32, 1000), (64, 777), (128, 301), (256, 40), (4, 1001),
                                           (8, 513), (48, 65), (2048, 70), (6144, 9), (300, 37),
                                           (1, 4099), (7, 301)])
def test_device_quantizer_matches_oracle(dev, orc, group, ngroups):
    rng = np.random.default_rng(group * 7 + ngroups)
    x = rng.standard_normal(group * ngroups).astype(np.float32)
    x *= rng.uniform(1e-4, 30.0, x.size).astype(np.float32)   # scales over 5 decades
    x[rng.integers(0, x.size, 40)] = 0.0
    if ngroups > 3:
        x[2 * group:3 * group] = 0.0                          # one all-zero group
    q, s = _quantize(dev, x, group)
    qo, so = orc.quantize_groupwise(x, group)
    tag = f"group={group} ngroups={ngroups}"
    np.testing.assert_array_equal(s.view(np.uint32), so.view(np.uint32), err_msg=tag)
    np.testing.assert_array_equal(q, qo, err_msg=tag)


@pytest.mark.parametrize("shift_x,shift_q", [(1, 0), (0, 1), (2, 3)])
def test_device_quantizer_unaligned_buffers(dev, orc, shift_x, shift_q):
    """Buffers off the 16-byte (x) / 4-byte (q) alignment of the float4 path."""
    torch, q3, _, _ = dev
    group, ngroups = 64, 150
    rng = np.random.default_rng(11 + shift_x + shift_q)
    x = rng.standard_normal(group * ngroups).astype(np.float32)
    xb = torch.zeros(x.size + 4, dtype=torch.float32, device="cuda")
    xd = xb[shift_x:shift_x + x.size]
    xd.copy_(torch.from_numpy(x))
    qb = torch.zeros(x.size + 4, dtype=torch.int8, device="cuda")
    qd = qb[shift_q:shift_q + x.size]
    q, s = q3.quantize_groupwise(xd, group, q=qd)
    torch.cuda.synchronize()
    qo, so = orc.quantize_groupwise(x, group)
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))
    np.testing.assert_array_equal(q.cpu().numpy(), qo)
    untouched = np.concatenate([qb.cpu().numpy()[:shift_q], qb.cpu().numpy()[shift_q + x.size:]])
    assert not untouched.any()


def test_device_quantizer_closed_forms(dev):
    # group g holds k (g + 1) with one element at +-127 (g + 1): s = g + 1, q = k
    rng = np.random.default_rng(8)
    ng, group = 40, 64
    k = rng.integers(-127, 128, size=(ng, group))
    k[:, 0] = np.where(rng.random(ng) < 0.5, 127, -127)
    rng.permuted(k, axis=1, out=k)
    x = (k * (np.arange(ng)[:, None] + 1)).astype(np.float32)
    # ties in group 0 (s = 1): n + 1/2 rounds to the even neighbour
    x[0, :6] = [0.5, 1.5, 2.5, -2.5, 126.5, 127.0]
    k[0, :6] = [0, 2, 2, -2, 126, 127]
    q, s = _quantize(dev, x, group)
    np.testing.assert_array_equal(s, np.arange(1, ng + 1, dtype=np.float32))
    np.testing.assert_array_equal(q.reshape(ng, group).astype(np.int64), k)


def test_device_quantizer_full_weight(dev, orc):
    """One full mlp up_proj [6144, 2048] at the model's group size."""
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((6144, 2048)) * 0.02).astype(np.float32)
    q, s = _quantize(dev, x, 64)
    qo, so = orc.quantize_groupwise(x, 64)
    np.testing.assert_array_equal(s.view(np.uint32), so.view(np.uint32))
    np.testing.assert_array_equal(q, qo)


def test_device_quantizer_rejects_partial_groups(dev):
    torch, q3, _, _ = dev
    x = torch.zeros(100, dtype=torch.float32, device="cuda")
    with pytest.raises(ValueError, match="whole groups"):
        q3.quantize_groupwise(x, 64)


def _hdr(ck, **kw):
    h = dict(vocab=SMALL["vocab"], hidden=SMALL["hidden"], intermediate=SMALL["inter"],
             layers=SMALL["layers"], heads=SMALL["heads"], kv_heads=SMALL["kv_heads"],
             max_position=262144, rope_theta=int(SMALL["theta"]), rms_eps=SMALL["eps"],
             vision_hidden=8, vision_depth=18, vision_patch=2, vision_spatial_merge=2,
             vision_temporal_patch=2, vision_heads=2, vision_intermediate=16,
             out_hidden=SMALL["hidden"], image_token_id=151655, vision_start_token_id=151652,
             vision_end_token_id=151653, video_token_id=151656, text_bits=8,
             group_size=SMALL["gs"], vision_bits=16, group_quantized=1)
    h.update(kw)
    return h


# checkpoint group -> (values, scales) keys of the test model arrays
PAIRS = {"embed": ("emb_w", "emb_s"), "attn_norm": ("anorm_w", "anorm_s"),
         "down": ("wd", "sd"), "gate": ("wg", "sg"), "up": ("wu", "su"),
         "mlp_norm": ("mnorm_w", "mnorm_s"), "k_norm": ("knorm_w", "knorm_s"),
         "k": ("wk", "sk"), "o": ("wo", "so"), "q_norm": ("qnorm_w", "qnorm_s"),
         "q": ("wq", "sq"), "v": ("wv", "sv"), "final_norm": ("fnorm_w", "fnorm_s")}
# q3vl_text_model pointer fields -> test model arrays
STRUCT_FIELDS = {"emb_w": "emb_w", "emb_s": "emb_s", "fnorm_w": "fnorm_w", "fnorm_s": "fnorm_s",
                 "anorm_w": "anorm_w", "anorm_s": "anorm_s", "mnorm_w": "mnorm_w",
                 "mnorm_s": "mnorm_s", "qnorm_w": "qnorm_w", "qnorm_s": "qnorm_s",
                 "knorm_w": "knorm_w", "knorm_s": "knorm_s",
                 **{w: w for w in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")},
                 **{s: s for s in ("sq", "sk", "sv", "so", "sg", "su", "sd")}}


def test_export_writes_the_oracle_quantized_file(dev, orc, tmp_path):
    torch, _, ck, _ = dev
    hdr = _hdr(ck, vocab=1024, hidden=256, intermediate=512, heads=2, kv_heads=1,
               out_hidden=256)
    rng = np.random.default_rng(10)
    floats = {n: (rng.standard_normal(s) * rng.uniform(0.01, 2.0)).astype(np.float32)
              for n, s in ck.text_shapes(hdr).items()}
    a, b = str(tmp_path / "device.bin"), str(tmp_path / "oracle.bin")
    ck.export_checkpoint(a, hdr, {n: torch.from_numpy(v).cuda() for n, v in floats.items()})
    ck.write_checkpoint(b, hdr, {n: orc.quantize_groupwise(v, ck.quant_group(hdr, n))
                                 for n, v in floats.items()})
    assert open(a, "rb").read() == open(b, "rb").read()


@pytest.fixture(scope="module")
def small_file(dev, tmp_path_factory):
    _, _, ck, _ = dev
    m = make_text_model(80, SMALL)
    hdr = _hdr(ck)
    path = str(tmp_path_factory.mktemp("ck") / "small.bin")
    ck.write_checkpoint(path, hdr, {n: (m[w], m[s]) for n, (w, s) in PAIRS.items()})
    return path, hdr, m


def test_load_places_the_file_bytes(dev, small_file):
    torch, _, ck, hip = dev
    path, hdr, m = small_file
    with ck.Checkpoint(path, max_seq=256) as c:
        assert c.header == ck.read_header(path)
        st = c.model.c
        for f in ("vocab", "hidden", "layers", "heads", "kv_heads", "max_seq"):
            assert getattr(st, f) == SMALL[f], f
        assert st.inter == SMALL["inter"] and st.head_dim == 128 and st.gs == SMALL["gs"]
        for field, key in STRUCT_FIELDS.items():
            want = np.ascontiguousarray(m[key])
            got = _d2h(hip, getattr(st, field), want.nbytes, want.dtype)
            np.testing.assert_array_equal(got, want.reshape(-1), err_msg=field)
            assert getattr(st, field) % 256 == 0, field
        cos, sin = ck.rope_tables(hdr["rope_theta"], 128, 256)
        np.testing.assert_array_equal(_d2h(hip, st.rope_cos, cos.nbytes, np.float32),
                                      cos.reshape(-1))
        np.testing.assert_array_equal(_d2h(hip, st.rope_sin, sin.nbytes, np.float32),
                                      sin.reshape(-1))


@pytest.mark.parametrize("ctx", [0, 100])
def test_decode_from_a_loaded_checkpoint(dev, orc, small_file, ctx):
    torch, q3, ck, _ = dev
    from q3vl_int8 import model as qm
    path, hdr, m = small_file
    max_seq = 256
    dims = dict(SMALL, max_seq=max_seq)
    arrays = dict(m)
    arrays["rope_cos"], arrays["rope_sin"] = ck.rope_tables(hdr["rope_theta"], 128, max_seq)
    k16, v16 = make_kv_cache(81 + ctx, dims, ctx)
    ko, vo = k16.view(np.uint16).copy(), v16.view(np.uint16).copy()
    with ck.Checkpoint(path, max_seq=max_seq) as c:
        kd = torch.from_numpy(k16.view(np.int16).copy()).cuda()
        vd = torch.from_numpy(v16.view(np.int16).copy()).cuda()
        token = 17
        tok = torch.tensor([token], dtype=torch.int32, device="cuda")
        pos = torch.tensor([ctx], dtype=torch.int32, device="cuda")
        logits = torch.zeros(dims["vocab"], dtype=torch.float32, device="cuda")
        ws = qm.alloc_decode_workspace(c.model)
        for step in range(4):
            qm.decode_step(c.model, kd, vd, tok, pos, logits, ws)
            torch.cuda.synchronize()
            nid, lo = orc.decode_step(dims, arrays, ko, vo, token, ctx + step, kv_fp16=True)
            tag = f"ctx={ctx} step={step} token={token}"
            np.testing.assert_array_equal(logits.cpu().numpy().view(np.uint32),
                                          lo.view(np.uint32), err_msg=tag)
            np.testing.assert_array_equal(kd.cpu().numpy().view(np.uint16), ko, err_msg=tag)
            np.testing.assert_array_equal(vd.cpu().numpy().view(np.uint16), vo, err_msg=tag)
            assert int(tok.item()) == nid and int(pos.item()) == ctx + step + 1, tag
            token = nid


def test_load_rejects_what_the_decode_step_cannot_serve(dev, tmp_path, small_file):
    torch, q3, ck, _ = dev
    path, hdr, m = small_file
    # truncated: the text groups end past the file
    blob = open(path, "rb").read()
    short = str(tmp_path / "short.bin")
    open(short, "wb").write(blob[:len(blob) // 2])
    with pytest.raises(q3.Q3VLError, match="text tensors end"):
        ck.Checkpoint(short, max_seq=256)
    # fp16 text weights: the file is valid, the decode step runs int8 only
    h16 = dict(hdr, text_bits=16)
    p16 = str(tmp_path / "fp16.bin")
    open(p16, "wb").write(ck.pack_header(h16) + b"\0" * 64)
    with pytest.raises(q3.Q3VLError, match="text_bits 16"):
        ck.Checkpoint(p16, max_seq=256)
    with pytest.raises(q3.Q3VLError, match="max_seq"):
        ck.Checkpoint(path, max_seq=0)


@pytest.mark.parametrize("gs", [32, 128])
def test_load_and_decode_other_group_sizes(dev, orc, tmp_path, gs):
    """A checkpoint exported at group 32 / 128 loads and decodes bit-exact."""
    torch, q3, ck, _ = dev
    from q3vl_int8 import model as qm
    dims = dict(SMALL, layers=1, gs=gs)
    m = make_text_model(120 + gs, dims)
    hdr = _hdr(ck, layers=1, group_size=gs)
    path = str(tmp_path / f"g{gs}.bin")
    ck.write_checkpoint(path, hdr, {n: (m[w], m[s]) for n, (w, s) in PAIRS.items()})
    arrays = dict(m)
    arrays["rope_cos"], arrays["rope_sin"] = ck.rope_tables(hdr["rope_theta"], 128, dims["max_seq"])
    k16, v16 = make_kv_cache(121 + gs, dims, 50)
    ko, vo = k16.view(np.uint16).copy(), v16.view(np.uint16).copy()
    with ck.Checkpoint(path, max_seq=dims["max_seq"]) as c:
        assert c.model.c.gs == gs
        kd = torch.from_numpy(k16.view(np.int16).copy()).cuda()
        vd = torch.from_numpy(v16.view(np.int16).copy()).cuda()
        token = 3
        tok = torch.tensor([token], dtype=torch.int32, device="cuda")
        pos = torch.tensor([50], dtype=torch.int32, device="cuda")
        logits = torch.zeros(dims["vocab"], dtype=torch.float32, device="cuda")
        ws = qm.alloc_decode_workspace(c.model)
        for step in range(2):
            qm.decode_step(c.model, kd, vd, tok, pos, logits, ws)
            torch.cuda.synchronize()
            nid, lo = orc.decode_step(dims, arrays, ko, vo, token, 50 + step, kv_fp16=True)
            np.testing.assert_array_equal(logits.cpu().numpy().view(np.uint32), lo.view(np.uint32))
            np.testing.assert_array_equal(kd.cpu().numpy().view(np.uint16), ko)
            assert int(tok.item()) == nid
            token = nid
