"""C ABI checks that need no GPU: the libraries load, export every function
include/q3vl_int8.h declares, and the host-only dispatch logic follows the
reference's linear() acceptance rules (matmul/src/cpu_wrapper.cpp:320-395)."""
import ctypes
import subprocess

import pytest

import q3vl_int8 as q


def test_library_exports_every_declared_function():
    lib = q.lib()
    names = q.header_functions()
    assert len(names) >= 15
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert lib.q3vl_abi_version() == 3


def test_linear_dropin_exports_cpp_linear():
    out = subprocess.run(["nm", "-DC", q.LINEAR_LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    assert "T linear(void const*, void const*, void const*, void const*, void const*, void*," in out
    ctypes.CDLL(q.LINEAR_LIB_PATH)  # loads (resolves libq3vl_int8.so via rpath)


@pytest.mark.parametrize("combo,ok", [
    ((q.FP32, q.INT8, q.FP32, q.FP32, 0, 1, 1), True),
    ((q.FP32, q.INT8, q.FP32, q.FP32, 1, 1, 1), False),   # bias rejected (:339)
    ((q.FP32, q.INT8, q.FP32, q.FP32, 0, 0, 1), False),   # row-quantized path
    ((q.FP32, q.INT8, q.FP32, q.FP32, 0, 1, 0), False),   # non-transposed B
    ((q.FP16, q.INT8, q.FP32, q.FP32, 0, 1, 1), False),
    ((q.FP32, q.FP16, q.FP32, q.FP32, 0, 1, 1), False),   # fp16 weights: not this path
    ((q.FP32, q.INT8, q.FP16, q.FP32, 0, 1, 1), False),
    ((q.FP32, q.INT8, q.FP32, q.FP16, 0, 1, 1), False),
])
def test_dtype_acceptance(combo, ok):
    rc = q.check_dtypes(*combo)
    assert (rc == q.OK) == ok
    if not ok:
        assert rc == q.ERR_UNSUPPORTED
        assert "not supported" in q.last_error()


def test_lane_path_rule():
    assert q.uses_lane_path(1, 1024, 1024)
    assert q.uses_lane_path(1, 151936, 2048)
    assert not q.uses_lane_path(1, 1000, 2048)
    assert not q.uses_lane_path(1, 2048, 512)
    assert not q.uses_lane_path(8, 151936, 2048)


def test_workspace_bytes_covers_shapes():
    small = q.workspace_bytes(1, 6144, 2048, 64)
    big = q.workspace_bytes(512, 12288, 2048, 64)
    assert 0 < small < big
    assert big >= 512 * 2048 * 2 + 512 * 32 * 4


def _fake_model(**over):
    """A q3vl_text_model whose tensors are fake (aligned, non-null) addresses:
    the decode step validates the model before touching any of them."""
    from golden.gen import SMALL
    from q3vl_int8 import model as qm
    dims = dict(SMALL, **over)
    return qm.make_struct(dims, lambda n: 0x100000)


@pytest.mark.parametrize("over,code,text", [
    (dict(max_seq=100), q.ERR_INVALID_ARGUMENT, "multiple of 8"),
    (dict(head_dim=64), q.ERR_UNSUPPORTED, "head_dim 128"),
    (dict(heads=32, kv_heads=8, hidden=4096), q.ERR_UNSUPPORTED, "heads/kv_heads"),
    (dict(max_seq=40000), q.ERR_UNSUPPORTED, "too long"),
    (dict(inter=1000), q.ERR_UNSUPPORTED, "[1024, 8192]"),
])
def test_decode_step_rejects_unsupported_models(over, code, text):
    lib = q.lib()
    s = _fake_model(**over)
    lib.q3vl_decode_step.restype = ctypes.c_int
    one = ctypes.c_void_p(0x200000)
    rc = lib.q3vl_decode_step(ctypes.byref(s), one, one, one, one, one, None, ctypes.c_size_t(0),
                              None)
    assert rc == code, q.last_error()
    assert text in q.last_error()


def test_static_decode_rejects_oversized_scratch():
    """q3vl_decode_step_static refuses a model whose decode scratch exceeds
    its static array, before any device work (so it runs without a GPU)."""
    from q3vl_int8 import model as qm
    L = q.lib()
    L.q3vl_decode_static_scratch_bytes.restype = ctypes.c_size_t
    cap = L.q3vl_decode_static_scratch_bytes()
    assert cap == 1 << 20
    dims = dict(vocab=151936, hidden=8192, inter=8192, layers=1, heads=64, kv_heads=64,
                head_dim=128, max_seq=4096, gs=64, eps=1e-6)
    fake = 1 << 20  # non-null, aligned, never dereferenced
    c = qm.make_struct(dims, lambda n: fake)
    assert qm.decode_workspace_bytes(type("M", (), {"c": c})()) > cap
    L.q3vl_decode_step_static.restype = ctypes.c_int
    L.q3vl_decode_step_static.argtypes = [ctypes.POINTER(qm.TextModelC)] + [ctypes.c_void_p] * 6
    rc = L.q3vl_decode_step_static(ctypes.byref(c), fake, fake, fake, fake, fake, None)
    assert rc == q.ERR_UNSUPPORTED
    assert "static scratch" in q.last_error()
