"""The GPU decode step (q3vl_decode_step through the C ABI) against the
oracle's decode step in its fp16-cache mode (oracle/decode_oracle.c, a
restatement of model/src/forward.cpp:458-720 pinned bit for bit against the
reference's compiled forward_text in tests/test_decode_oracle.py).

Bar: logits, every K/V cache row and the greedy ids bit-exact; the step
reads token and pos from device memory and advances both there.
"""
import numpy as np
import pytest

from golden.gen import QWEN3VL_2B, SMALL, make_kv_cache, make_text_model

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from q3vl_int8 import model as qm
    return torch, qm


class Stepper:
    """Device and oracle copies of one model + caches, stepped together."""

    def __init__(self, dev, orc, dims, seed, ctx, token, stale_nan=False, qscale=1.0):
        torch, qm = dev
        self.torch, self.qm, self.orc, self.dims = torch, qm, orc, dims
        self.m = make_text_model(seed, dims)
        if qscale != 1.0:  # larger queries through the q-norm's group scales
            self.m["qnorm_s"] = (self.m["qnorm_s"] * np.float32(qscale)).astype(np.float32)
        k16, v16 = make_kv_cache(seed + 1, dims, ctx)
        if stale_nan:  # rows at and past ctx hold NaN bits, as an unwritten cache may
            k16[:, :, ctx:] = np.float16("nan")
            v16[:, :, ctx:] = np.float16("nan")
        self.ko, self.vo = k16.view(np.uint16).copy(), v16.view(np.uint16).copy()
        self.model = qm.DeviceTextModel(dims, self.m)
        self.kd = torch.from_numpy(k16.view(np.int16).copy()).cuda()
        self.vd = torch.from_numpy(v16.view(np.int16).copy()).cuda()
        self.tok = torch.tensor([token], dtype=torch.int32, device="cuda")
        self.pos = torch.tensor([ctx], dtype=torch.int32, device="cuda")
        self.logits = torch.zeros(dims["vocab"], dtype=torch.float32, device="cuda")
        self.ws = qm.alloc_decode_workspace(self.model)
        self.token, self.p = token, ctx

    def step(self):
        torch = self.torch
        self.qm.decode_step(self.model, self.kd, self.vd, self.tok, self.pos, self.logits,
                            self.ws)
        torch.cuda.synchronize()
        nid, lo = self.orc.decode_step(self.dims, self.m, self.ko, self.vo, self.token, self.p,
                                       kv_fp16=True, chunked=self.dims.get("attn_order", 0) == 1)
        lg = self.logits.cpu().numpy()
        tag = f"pos={self.p} token={self.token}"
        np.testing.assert_array_equal(lg.view(np.uint32), lo.view(np.uint32), err_msg=tag)
        np.testing.assert_array_equal(self.kd.cpu().numpy().view(np.uint16), self.ko, err_msg=tag)
        np.testing.assert_array_equal(self.vd.cpu().numpy().view(np.uint16), self.vo, err_msg=tag)
        assert int(self.tok.item()) == nid, tag
        assert int(self.pos.item()) == self.p + 1, tag
        self.token, self.p = nid, self.p + 1
        return nid


def test_decode_chained_steps_small(dev, orc):
    s = Stepper(dev, orc, dict(SMALL), seed=21, ctx=100, token=7)
    for _ in range(4):
        s.step()


@pytest.mark.parametrize("pos", [0, 7, 8, 63, 64, 255])
def test_decode_edge_positions(dev, orc, pos):
    dims = dict(SMALL, layers=1)
    Stepper(dev, orc, dims, seed=30 + pos, ctx=pos, token=pos % 4096).step()


@pytest.mark.parametrize("pos", [511, 512, 1023, 1024, 1100, 1535, 1536])
def test_decode_context_past_one_value_chunk(dev, orc, pos):
    """Contexts of 512 to 1537 positions, on either side of 512, 1024 and
    1536: the value-weighted sum stages V through LDS in chunks of 1024
    positions."""
    dims = dict(SMALL, layers=1, max_seq=1600)
    Stepper(dev, orc, dims, seed=40, ctx=pos, token=11).step()


@pytest.mark.parametrize("pos", [1000, 2100])
def test_decode_stale_rows_past_the_context(dev, orc, pos):
    """Cache rows at and past pos hold NaN bits (never written): the step
    reads no row past pos into its result and overwrites the row at pos.
    pos=2100 spans three score passes and three value chunks."""
    dims = dict(SMALL, layers=1, max_seq=2304)
    Stepper(dev, orc, dims, seed=45, ctx=pos, token=5, stale_nan=True).step()


def test_decode_position_out_of_range(dev):
    """*pos = max_seq has no cache row: the caches stay as they were and the
    logits are NaN."""
    torch, qm = dev
    dims = dict(SMALL, layers=1, max_seq=256)
    m = make_text_model(70, dims)
    k16, v16 = make_kv_cache(71, dims, 256)
    model = qm.DeviceTextModel(dims, m)
    kd = torch.from_numpy(k16.view(np.int16).copy()).cuda()
    vd = torch.from_numpy(v16.view(np.int16).copy()).cuda()
    tok = torch.tensor([9], dtype=torch.int32, device="cuda")
    pos = torch.tensor([256], dtype=torch.int32, device="cuda")
    logits = torch.zeros(dims["vocab"], dtype=torch.float32, device="cuda")
    qm.decode_step(model, kd, vd, tok, pos, logits, qm.alloc_decode_workspace(model))
    torch.cuda.synchronize()
    assert torch.isnan(logits).all()
    np.testing.assert_array_equal(kd.cpu().numpy(), k16.view(np.int16))
    np.testing.assert_array_equal(vd.cpu().numpy(), v16.view(np.int16))


@pytest.mark.parametrize("gs,token", [(64, -1), (64, 4096), (32, 4096)])
def test_decode_token_out_of_range(dev, gs, token):
    """A token outside [0, vocab) reads no table row: its embedding is a NaN
    row, so the logits are NaN, the greedy id is 0 (NaN never wins), the
    cache rows at pos hold NaN and every other row is untouched (group 64,
    the decode step's, and 32)."""
    torch, qm = dev
    dims = dict(SMALL, layers=1, gs=gs)
    m = make_text_model(75, dims)
    k16, v16 = make_kv_cache(76, dims, 100)
    model = qm.DeviceTextModel(dims, m)
    kd = torch.from_numpy(k16.view(np.int16).copy()).cuda()
    vd = torch.from_numpy(v16.view(np.int16).copy()).cuda()
    tok = torch.tensor([token], dtype=torch.int32, device="cuda")
    pos = torch.tensor([100], dtype=torch.int32, device="cuda")
    logits = torch.zeros(dims["vocab"], dtype=torch.float32, device="cuda")
    qm.decode_step(model, kd, vd, tok, pos, logits, qm.alloc_decode_workspace(model))
    torch.cuda.synchronize()
    assert torch.isnan(logits).all()
    assert int(tok.item()) == 0 and int(pos.item()) == 101
    for got, ref in ((kd, k16), (vd, v16)):
        g = got.cpu().numpy().view(np.float16)
        assert np.isnan(g[:, :, 100]).all()
        keep = np.ones(g.shape[2], bool)
        keep[100] = False
        np.testing.assert_array_equal(g[:, :, keep].view(np.uint16), ref[:, :, keep].view(np.uint16))


@pytest.mark.parametrize("gs", [32, 128])
def test_decode_other_group_sizes(dev, orc, gs):
    """The exporter's other group sizes (export_qwen_bin.py:371): every GEMV,
    the fused norms and the head norms at groups of 32 and 128."""
    s = Stepper(dev, orc, dict(SMALL, layers=1, gs=gs), seed=90 + gs, ctx=100, token=9)
    for _ in range(3):
        s.step()


def test_decode_three_query_heads_per_kv_head(dev, orc):
    dims = dict(SMALL, layers=1, heads=24, kv_heads=8, hidden=3072, inter=1024)
    Stepper(dev, orc, dims, seed=50, ctx=70, token=3).step()


def test_decode_full_config_step(dev, orc):
    """One step of the full Qwen3-VL-2B text decoder (28 layers, vocab
    151936) at context 1024 with random weights, the benchmarked workload."""
    print("full-size decode step: building model", flush=True)
    dims = dict(QWEN3VL_2B, max_seq=1088)
    s = Stepper(dev, orc, dims, seed=60, ctx=1024, token=151000)
    print("full-size decode step: stepping", flush=True)
    s.step()


# ---------------------------------------------- the chunked attention order
# Q3VL_ATTN_CHUNKED (no counterpart in the reference): checked bit for bit
# against the oracle's restatement of that order (orc_attention_chunked),
# whose own distance from the reference order is pinned on the CPU.
CHUNKED = 1


@pytest.mark.parametrize("pos", [0, 7, 63, 64, 65, 127, 255])
def test_decode_chunked_edge_positions(dev, orc, pos):
    dims = dict(SMALL, layers=1, attn_order=CHUNKED)
    Stepper(dev, orc, dims, seed=130 + pos, ctx=pos, token=pos % 4096).step()


def test_decode_chunked_chained_steps(dev, orc):
    s = Stepper(dev, orc, dict(SMALL, attn_order=CHUNKED), seed=121, ctx=126, token=7)
    for _ in range(4):  # crosses the chunk boundary at 128
        s.step()


@pytest.mark.parametrize("pos", [1000, 2100])
def test_decode_chunked_stale_rows_past_the_context(dev, orc, pos):
    dims = dict(SMALL, layers=1, max_seq=2304, attn_order=CHUNKED)
    Stepper(dev, orc, dims, seed=145, ctx=pos, token=5, stale_nan=True).step()


def test_decode_chunked_three_query_heads_per_kv_head(dev, orc):
    dims = dict(SMALL, layers=1, heads=24, kv_heads=8, hidden=3072, inter=1024, attn_order=CHUNKED)
    Stepper(dev, orc, dims, seed=150, ctx=200, token=3).step()


def test_decode_chunked_full_config_step(dev, orc):
    print("full-size chunked decode step: building model", flush=True)
    dims = dict(QWEN3VL_2B, max_seq=1088, attn_order=CHUNKED)
    s = Stepper(dev, orc, dims, seed=160, ctx=1024, token=151000)
    print("full-size chunked decode step: stepping", flush=True)
    s.step()


@pytest.mark.parametrize("order", [0, CHUNKED])
@pytest.mark.parametrize("qscale", [15.0, 100.0])
def test_decode_wide_score_range(dev, orc, order, qscale):
    """Queries scaled up by the q-norm's scales, so a head's scores (about
    qscale * N(0, 1) against the N(0, 1) cache) spread past exp256's range:
    at 15 over the context (~90) but mostly not within one 64-position chunk
    (~70), at 100 within chunks too. The reference zeroes a head once some
    exp256(s - M) is -inf (text_layer.cpp:512-515); both orders must zero
    exactly those heads (the chunked order through each chunk's smallest
    finite score), bit for bit against the oracle."""
    dims = dict(SMALL, layers=1, max_seq=1088, attn_order=order)
    Stepper(dev, orc, dims, seed=180, ctx=1000, token=9, qscale=qscale).step()


def test_decode_chunked_position_out_of_range(dev):
    """*pos = max_seq: caches untouched, logits NaN, as in the reference order."""
    torch, qm = dev
    dims = dict(SMALL, layers=1, max_seq=256, attn_order=CHUNKED)
    m = make_text_model(170, dims)
    k16, v16 = make_kv_cache(171, dims, 256)
    model = qm.DeviceTextModel(dims, m)
    kd = torch.from_numpy(k16.view(np.int16).copy()).cuda()
    vd = torch.from_numpy(v16.view(np.int16).copy()).cuda()
    tok = torch.tensor([9], dtype=torch.int32, device="cuda")
    pos = torch.tensor([256], dtype=torch.int32, device="cuda")
    logits = torch.zeros(dims["vocab"], dtype=torch.float32, device="cuda")
    qm.decode_step(model, kd, vd, tok, pos, logits, qm.alloc_decode_workspace(model))
    torch.cuda.synchronize()
    assert torch.isnan(logits).all()
    np.testing.assert_array_equal(kd.cpu().numpy(), k16.view(np.int16))
    np.testing.assert_array_equal(vd.cpu().numpy(), v16.view(np.int16))
