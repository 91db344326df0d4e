"""q3vl_decode_step_static, the decode step that allocates nothing (its
scratch is a static device array), against q3vl_decode_step with a caller
workspace: logits, next token, position and both caches bit-identical, on
two calls in a row, the second with a smaller model."""
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


def test_static_scratch_decode_matches_workspace_decode():
    cap = qm.static_scratch_bytes()
    sizes = []
    for dims, seed, ctx, token, steps in [(dict(SMALL), 61, 100, 7, 2), (TINY, 62, 20, 3, 1)]:
        ref = _state(dims, seed, ctx, token)
        got = _state(dims, seed, ctx, token)
        need = qm.decode_workspace_bytes(ref[0])
        assert need <= cap
        sizes.append(need)
        ws = qm.alloc_decode_workspace(ref[0])
        for s in range(steps):
            qm.decode_step(*ref[:6], ws)
            qm.decode_step_static(*got)
            torch.cuda.synchronize()
            what = f"{dims['layers']}-layer model, step {s}"
            assert np.array_equal(got[5].cpu().numpy().view(np.uint32),
                                  ref[5].cpu().numpy().view(np.uint32)), f"logits differ: {what}"
            assert int(got[3].item()) == int(ref[3].item()), f"token differs: {what}"
            assert int(got[4].item()) == int(ref[4].item()) == ctx + s + 1, f"pos differs: {what}"
            assert torch.equal(got[1], ref[1]) and torch.equal(got[2], ref[2]), f"caches: {what}"
    assert sizes[1] < sizes[0]  # the second call's input is the smaller one
