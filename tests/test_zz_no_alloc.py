"""q3vl_decode_step_static, the decode step that allocates nothing (its
scratch is a static device array), against q3vl_decode_step with a caller
workspace: logits, next token, position and both caches bit-identical, on
two calls in a row, the second with a smaller model, in both attention
orders (the chunked order carves its per-chunk partials from the same
array); device free memory unchanged across every static call after the
first; and a first call for a shape never seen before made under HIP graph
capture, then replayed."""
import numpy as np
import pytest

from golden.gen import SMALL, make_kv_cache, make_text_model

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from q3vl_int8 import model as qm  # noqa: E402

TINY = dict(vocab=1024, hidden=1024, inter=1024, layers=1, heads=8, kv_heads=8, head_dim=128,
            max_seq=64, gs=64, eps=1e-6, theta=5000000.0)


def _state(dims, seed, ctx, token):
    m = make_text_model(seed, dims)
    k16, v16 = make_kv_cache(seed + 1, dims, ctx)
    dm = qm.DeviceTextModel(dims, m)
    kd = torch.from_numpy(k16.view(np.int16).copy()).cuda()
    vd = torch.from_numpy(v16.view(np.int16).copy()).cuda()
    tok = torch.tensor([token], dtype=torch.int32, device="cuda")
    pos = torch.tensor([ctx], dtype=torch.int32, device="cuda")
    logits = torch.full((dims["vocab"],), float("nan"), dtype=torch.float32, device="cuda")
    return dm, kd, vd, tok, pos, logits


def _free_bytes():
    torch.cuda.synchronize()
    return torch.cuda.mem_get_info()[0]


@pytest.mark.parametrize("order", [0, 1], ids=["reference_order", "chunked_order"])
def test_static_scratch_decode_matches_workspace_decode(order):
    cap = qm.static_scratch_bytes()
    sizes = []
    first = True
    for dims, seed, ctx, token, steps in [(dict(SMALL), 61, 100, 7, 2), (TINY, 62, 20, 3, 1)]:
        dims = dict(dims, attn_order=order)
        ref = _state(dims, seed, ctx, token)
        got = _state(dims, seed, ctx, token)
        need = qm.decode_workspace_bytes(ref[0])
        assert need <= cap
        sizes.append(need)
        ws = qm.alloc_decode_workspace(ref[0])
        for s in range(steps):
            qm.decode_step(*ref[:6], ws)
            free0 = _free_bytes()
            qm.decode_step_static(*got)
            free1 = _free_bytes()
            if not first:  # (the first call may load code on the device)
                assert free1 == free0, f"device memory changed by {free0 - free1} bytes"
            first = False
            what = f"{dims['layers']}-layer model, step {s}"
            assert np.array_equal(got[5].cpu().numpy().view(np.uint32),
                                  ref[5].cpu().numpy().view(np.uint32)), f"logits differ: {what}"
            assert int(got[3].item()) == int(ref[3].item()), f"token differs: {what}"
            assert int(got[4].item()) == int(ref[4].item()) == ctx + s + 1, f"pos differs: {what}"
            assert torch.equal(got[1], ref[1]) and torch.equal(got[2], ref[2]), f"caches: {what}"
    assert sizes[1] < sizes[0]  # the second call's input is the smaller one


@pytest.mark.parametrize("order", [0, 1], ids=["reference_order", "chunked_order"])
def test_static_first_call_under_graph_capture(order):
    """The first static call for a shape no other test uses (hidden 1536 or
    1280, 16 query and 8 KV heads) is made under HIP graph capture; one
    replay equals one workspace decode step bit for bit."""
    hidden = 1536 if order == 0 else 1280
    dims = dict(TINY, hidden=hidden, inter=hidden, heads=16, kv_heads=8, max_seq=128, attn_order=order)
    seed, ctx, token = 64 + order, 40, 11
    got = _state(dims, seed, ctx, token)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        qm.decode_step_static(*got)
    g.replay()
    torch.cuda.synchronize()
    ref = _state(dims, seed, ctx, token)
    qm.decode_step(*ref[:6], qm.alloc_decode_workspace(ref[0]))
    torch.cuda.synchronize()
    assert np.array_equal(got[5].cpu().numpy().view(np.uint32), ref[5].cpu().numpy().view(np.uint32))
    assert int(got[3].item()) == int(ref[3].item())
    assert int(got[4].item()) == int(ref[4].item()) == ctx + 1
    assert torch.equal(got[1], ref[1]) and torch.equal(got[2], ref[2])
