"""q3vl_int8 -- Python binding of libq3vl_int8.so, the MI355X int8 matmul path.

ctypes over the C ABI declared in include/q3vl_int8.h. torch tensors are used
only as device buffers (pointers, shapes, the current HIP stream). Every
function raises Q3VLError with the library's message on a non-zero status and
fails loudly when the library is absent: there is no CPU fallback.

Names and argument meanings mirror the reference engine's matmul entry
linear() (matmul/src/cpu_wrapper.cpp:308-396) restricted to its int8
group-quantized branch, plus its decode-path consumers swiglu
(layers/src/text_layer.cpp:420-434) and greedy_decode
(tokenizer/src/utils.cpp:34-44).
"""
from __future__ import annotations

import ctypes
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libq3vl_int8.so")
LINEAR_LIB_PATH = os.path.join(_HERE, "libq3vl_linear.so")
HEADER_PATH = os.path.join(os.path.dirname(os.path.dirname(_HERE)), "include", "q3vl_int8.h")

OK, ERR_INVALID_ARGUMENT, ERR_UNSUPPORTED, ERR_HIP, ERR_OUT_OF_MEMORY = 0, 1, 2, 3, 4
FP32, INT32, FP16, INT8, INT4 = 0, 1, 2, 3, 4


class Q3VLError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"q3vl status {code}: {msg}")
        self.code = code


_lib = None
_sz = ctypes.c_size_t
_vp = ctypes.c_void_p


def _declare(lib):
    i = ctypes.c_int
    sigs = {
        "q3vl_last_error": (ctypes.c_char_p, []),
        "q3vl_abi_version": (i, []),
        "q3vl_workspace_bytes": (_sz, [_sz, _sz, _sz, _sz]),
        "q3vl_check_dtypes": (i, [i, i, i, i, i, i, i]),
        "q3vl_uses_lane_path": (i, [_sz, _sz, _sz]),
        "q3vl_quantize_rows": (i, [_vp, _vp, _vp, _sz, _sz, _sz, _vp]),
        "q3vl_linear_i8": (i, [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _vp, _sz, _vp]),
        "q3vl_linear_i8_groups": (i, [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _vp, _sz, _vp]),
        "q3vl_linear_i8_multi": (i, [_vp, _sz, _sz, _sz, i, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
        "q3vl_linear_i8_swiglu": (i, [_vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _vp, _sz, _vp]),
        "q3vl_mlp_i8": (i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _vp, _sz, _vp]),
        "q3vl_mlp_workspace_bytes": (_sz, [_sz, _sz, _sz, _sz]),
        "q3vl_lm_head_argmax": (i, [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _vp, _sz, _vp]),
        "q3vl_argmax_rows": (i, [_vp, _vp, _sz, _sz, _vp, _sz, _vp]),
        "q3vl_swiglu": (i, [_vp, _vp, _sz, _vp]),
        "q3vl_weight_register": (i, [_vp, _vp, _sz, _sz, _sz, _vp, _vp]),
        "q3vl_weight_lookup": (i, [_vp, _vp, _sz, _sz, _sz, _vp, _vp]),
        "q3vl_weight_release": (i, [_vp]),
        "q3vl_weight_release_all": (i, []),
        "q3vl_quantize_groupwise": (i, [_vp, _sz, _sz, _vp, _vp, _vp]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


def lib():
    """Load libq3vl_int8.so (raises OSError if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise OSError(f"{LIB_PATH} is missing: build it with `make -C {os.path.dirname(_HERE)}`")
        l = ctypes.CDLL(LIB_PATH)
        _declare(l)
        _lib = l
    return _lib


def header_functions(path: str = HEADER_PATH) -> list[str]:
    """Names of the functions declared in include/q3vl_int8.h."""
    text = open(path).read()
    return sorted(set(re.findall(r"\b(q3vl_[a-z0-9_]+)\s*\(", text)))


def _check(rc: int):
    if rc != OK:
        raise Q3VLError(rc, lib().q3vl_last_error().decode())


def last_error() -> str:
    return lib().q3vl_last_error().decode()


def check_dtypes(ta, tb, tb_scale, tc, has_bias, group_quantized, b_transpose) -> int:
    return lib().q3vl_check_dtypes(ta, tb, tb_scale, tc, int(has_bias), int(group_quantized),
                                   int(b_transpose))


def uses_lane_path(M, N, K) -> bool:
    return bool(lib().q3vl_uses_lane_path(M, N, K))


def workspace_bytes(M, N, K, gs) -> int:
    return lib().q3vl_workspace_bytes(M, N, K, gs)


# ---------------------------------------------------------------- torch glue
def _torch():
    import torch
    return torch


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    torch = _torch()
    s = torch.cuda.current_stream() if stream is None else stream
    return ctypes.c_void_p(s.cuda_stream)


def _need(t, dtype, name, ndim=None):
    torch = _torch()
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"{name} must have {ndim} dims")


def _ws(workspace):
    if workspace is None:
        return None, 0
    return ctypes.c_void_p(workspace.data_ptr()), workspace.numel() * workspace.element_size()


def alloc_workspace(M, N, K, gs, device="cuda"):
    """Device workspace for the linear entry points at shape (M, N, K)."""
    torch = _torch()
    return torch.zeros(workspace_bytes(M, N, K, gs), dtype=torch.uint8, device=device)


def quantize_rows(A, gs, q=None, a_s=None, stream=None):
    """Activation quantizer: A [M,K] fp32 -> (q int16 [M,K], a_s fp32 [M,K/gs])."""
    torch = _torch()
    _need(A, torch.float32, "A", 2)
    M, K = A.shape
    q = torch.empty((M, K), dtype=torch.int16, device=A.device) if q is None else q
    a_s = torch.empty((M, K // gs), dtype=torch.float32, device=A.device) if a_s is None else a_s
    _check(lib().q3vl_quantize_rows(_ptr(A), _ptr(q), _ptr(a_s), M, K, gs, _stream(stream)))
    return q, a_s


def linear_i8(A, W, S, gs, out=None, groups=None, workspace=None, stream=None):
    """C = A W^T with the reference's int8 numerics. A [M,K] f32, W [N,K] i8,
    S [N,K/gs] f32. groups (int32 [M,N,K/gs]) receives the exact group sums."""
    torch = _torch()
    _need(A, torch.float32, "A", 2)
    _need(W, torch.int8, "W", 2)
    _need(S, torch.float32, "S")
    M, K = A.shape
    N = W.shape[0]
    if W.shape[1] != K or S.numel() != N * (K // gs):
        raise ValueError("shape mismatch between A, W and S")
    out = torch.empty((M, N), dtype=torch.float32, device=A.device) if out is None else out
    _need(out, torch.float32, "out")
    wp, wb = _ws(workspace)
    if groups is None:
        rc = lib().q3vl_linear_i8(_ptr(A), _ptr(W), _ptr(S), _ptr(out), M, N, K, gs, wp, wb,
                                  _stream(stream))
    else:
        _need(groups, torch.int32, "groups")
        rc = lib().q3vl_linear_i8_groups(_ptr(A), _ptr(W), _ptr(S), _ptr(out), _ptr(groups), M,
                                         N, K, gs, wp, wb, _stream(stream))
    _check(rc)
    return out


def linear_i8_multi(A, Ws, Ss, gs, outs=None, workspace=None, stream=None):
    """Up to three linears sharing one activation: [A W_i^T for each i]."""
    torch = _torch()
    _need(A, torch.float32, "A", 2)
    M, K = A.shape
    n = len(Ws)
    Ns = [w.shape[0] for w in Ws]
    if outs is None:
        outs = [torch.empty((M, N), dtype=torch.float32, device=A.device) for N in Ns]
    PA = ctypes.c_void_p * n
    wp, wb = _ws(workspace)
    rc = lib().q3vl_linear_i8_multi(
        _ptr(A), M, K, gs, n, PA(*[w.data_ptr() for w in Ws]), PA(*[s.data_ptr() for s in Ss]),
        PA(*[o.data_ptr() for o in outs]), (ctypes.c_size_t * n)(*Ns), wp, wb, _stream(stream))
    _check(rc)
    return outs


def linear_i8_swiglu(A, Wg, Sg, Wu, Su, gs, out=None, workspace=None, stream=None):
    """H = silu(A Wg^T) * (A Wu^T)."""
    torch = _torch()
    _need(A, torch.float32, "A", 2)
    M, K = A.shape
    N = Wg.shape[0]
    out = torch.empty((M, N), dtype=torch.float32, device=A.device) if out is None else out
    wp, wb = _ws(workspace)
    rc = lib().q3vl_linear_i8_swiglu(_ptr(A), _ptr(Wg), _ptr(Sg), _ptr(Wu), _ptr(Su), _ptr(out),
                                     M, N, K, gs, wp, wb, _stream(stream))
    _check(rc)
    return out


def mlp_workspace_bytes(M, H, I, gs) -> int:
    return lib().q3vl_mlp_workspace_bytes(M, H, I, gs)


def mlp_i8(A, Wg, Sg, Wu, Su, Wd, Sd, gs, out=None, workspace=None, stream=None):
    """The MLP block: Y = (silu(A Wg^T) * (A Wu^T)) Wd^T, A [M,H], Wg/Wu [I,H],
    Wd [H,I]."""
    torch = _torch()
    _need(A, torch.float32, "A", 2)
    for t, n in ((Wg, "Wg"), (Wu, "Wu"), (Wd, "Wd")):
        _need(t, torch.int8, n, 2)
    for t, n in ((Sg, "Sg"), (Su, "Su"), (Sd, "Sd")):
        _need(t, torch.float32, n)
    M, H = A.shape
    I = Wg.shape[0]
    if Wg.shape != (I, H) or Wu.shape != (I, H) or Wd.shape != (H, I):
        raise ValueError("shape mismatch between A, Wg, Wu and Wd")
    out = torch.empty((M, H), dtype=torch.float32, device=A.device) if out is None else out
    _need(out, torch.float32, "out")
    wp, wb = _ws(workspace)
    _check(lib().q3vl_mlp_i8(_ptr(A), _ptr(Wg), _ptr(Sg), _ptr(Wu), _ptr(Su), _ptr(Wd), _ptr(Sd),
                             _ptr(out), M, H, I, gs, wp, wb, _stream(stream)))
    return out


def lm_head_argmax(A, W, S, gs, logits=None, ids=None, workspace=None, stream=None):
    """ids[m] = greedy_decode(A[m] W^T); optionally stores the logits."""
    torch = _torch()
    _need(A, torch.float32, "A", 2)
    M, K = A.shape
    V = W.shape[0]
    ids = torch.empty((M,), dtype=torch.int32, device=A.device) if ids is None else ids
    wp, wb = _ws(workspace)
    rc = lib().q3vl_lm_head_argmax(_ptr(A), _ptr(W), _ptr(S), _ptr(logits), _ptr(ids), M, V, K,
                                   gs, wp, wb, _stream(stream))
    _check(rc)
    return ids


def argmax_rows(logits, ids=None, workspace=None, stream=None):
    torch = _torch()
    _need(logits, torch.float32, "logits", 2)
    M, V = logits.shape
    ids = torch.empty((M,), dtype=torch.int32, device=logits.device) if ids is None else ids
    wp, wb = _ws(workspace)
    _check(lib().q3vl_argmax_rows(_ptr(logits), _ptr(ids), M, V, wp, wb, _stream(stream)))
    return ids


def swiglu(gate, up, stream=None):
    """In place: gate = silu(gate) * up."""
    torch = _torch()
    _need(gate, torch.float32, "gate")
    _need(up, torch.float32, "up")
    _check(lib().q3vl_swiglu(_ptr(gate), _ptr(up), gate.numel(), _stream(stream)))
    return gate


def quantize_groupwise(x, group, q=None, scales=None, stream=None):
    """The checkpoint exporter's weight quantizer on the device
    (export_bin/export_qwen_bin.py:260-275): x fp32 (any shape, numel a
    multiple of group) -> (q int8 like x, scales fp32 [numel/group])."""
    torch = _torch()
    _need(x, torch.float32, "x")
    n = x.numel()
    if group <= 0 or n % group:
        raise ValueError(f"{n} values are not whole groups of {group}")
    q = torch.empty(x.shape, dtype=torch.int8, device=x.device) if q is None else q
    scales = (torch.empty((n // group,), dtype=torch.float32, device=x.device)
              if scales is None else scales)
    _need(q, torch.int8, "q")
    _need(scales, torch.float32, "scales")
    if q.numel() != n or scales.numel() != n // group:
        raise ValueError("q / scales sizes do not match x")
    _check(lib().q3vl_quantize_groupwise(_ptr(x), n, group, _ptr(q), _ptr(scales),
                                         _stream(stream)))
    return q, scales
