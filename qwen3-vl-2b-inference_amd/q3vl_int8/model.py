"""ctypes layout of q3vl_text_model (include/q3vl_int8.h) and the decode-step
binding. The CPU checkers (orc_model, ref_model_desc) share this layout."""
from __future__ import annotations

import ctypes

_vp = ctypes.c_void_p

FIELD_ORDER = [
    ("emb_w", "emb_s"), ("fnorm_w", "fnorm_s"), ("anorm_w", "anorm_s"), ("mnorm_w", "mnorm_s"),
    ("qnorm_w", "qnorm_s"), ("knorm_w", "knorm_s"),
]
LINEAR_W = ["wq", "wk", "wv", "wo", "wg", "wu", "wd"]
LINEAR_S = ["sq", "sk", "sv", "so", "sg", "su", "sd"]


class TextModelC(ctypes.Structure):
    _fields_ = ([(n, ctypes.c_int) for n in ("vocab", "hidden", "inter", "layers", "heads",
                                             "kv_heads", "head_dim", "max_seq", "gs")]
                + [("eps", ctypes.c_float)]
                + [(n, _vp) for pair in FIELD_ORDER for n in pair]
                + [(n, _vp) for n in LINEAR_W] + [(n, _vp) for n in LINEAR_S]
                + [("rope_cos", _vp), ("rope_sin", _vp)]
                + [("attn_order", ctypes.c_int)])

ATTN_REFERENCE = 0  # Q3VL_ATTN_REFERENCE
ATTN_CHUNKED = 1    # Q3VL_ATTN_CHUNKED


def make_struct(dims: dict, ptr) -> TextModelC:
    """Fills the struct from dims and ptr(name) -> address for every tensor."""
    s = TextModelC()
    for n in ("vocab", "hidden", "inter", "layers", "heads", "kv_heads", "head_dim", "max_seq", "gs"):
        setattr(s, n, int(dims[n]))
    s.eps = float(dims["eps"])
    for pair in FIELD_ORDER:
        for n in pair:
            setattr(s, n, ptr(n))
    for n in LINEAR_W + LINEAR_S + ["rope_cos", "rope_sin"]:
        setattr(s, n, ptr(n))
    s.attn_order = int(dims.get("attn_order", ATTN_REFERENCE))
    return s


class DeviceTextModel:
    """A text model resident in device memory (torch tensors as buffers)."""

    def __init__(self, dims: dict, arrays: dict, device="cuda"):
        import torch
        self.dims = dict(dims)
        self.t = {k: torch.from_numpy(v).to(device) for k, v in arrays.items()}
        self.c = make_struct(dims, lambda n: self.t[n].data_ptr())

    @classmethod
    def from_device(cls, dims: dict, tensors: dict):
        self = cls.__new__(cls)
        self.dims = dict(dims)
        self.t = tensors
        self.c = make_struct(dims, lambda n: self.t[n].data_ptr())
        return self


def decode_workspace_bytes(model: DeviceTextModel) -> int:
    from . import lib
    L = lib()
    L.q3vl_decode_workspace_bytes.restype = ctypes.c_size_t
    L.q3vl_decode_workspace_bytes.argtypes = [ctypes.POINTER(TextModelC)]
    return L.q3vl_decode_workspace_bytes(ctypes.byref(model.c))


def decode_step(model: DeviceTextModel, k_cache, v_cache, token, pos, logits=None,
                workspace=None, stream=None):
    """One decode step on device state: reads token at *pos, writes the next
    token into `token` and increments `pos` (both int32 device tensors)."""
    from . import _check, _ptr, _stream, _ws, lib
    L = lib()
    L.q3vl_decode_step.restype = ctypes.c_int
    L.q3vl_decode_step.argtypes = [ctypes.POINTER(TextModelC), _vp, _vp, _vp, _vp, _vp, _vp,
                                   ctypes.c_size_t, _vp]
    wp, wb = _ws(workspace)
    _check(L.q3vl_decode_step(ctypes.byref(model.c), _ptr(k_cache), _ptr(v_cache), _ptr(token),
                              _ptr(pos), _ptr(logits), wp, wb, _stream(stream)))


def decode_step_static(model: DeviceTextModel, k_cache, v_cache, token, pos, logits=None,
                       stream=None):
    """decode_step with the library's static device scratch instead of a
    workspace: allocates nothing. Calls that overlap on one device race."""
    from . import _check, _ptr, _stream, lib
    L = lib()
    L.q3vl_decode_step_static.restype = ctypes.c_int
    L.q3vl_decode_step_static.argtypes = [ctypes.POINTER(TextModelC), _vp, _vp, _vp, _vp, _vp, _vp]
    _check(L.q3vl_decode_step_static(ctypes.byref(model.c), _ptr(k_cache), _ptr(v_cache),
                                     _ptr(token), _ptr(pos), _ptr(logits), _stream(stream)))


def static_scratch_bytes() -> int:
    from . import lib
    L = lib()
    L.q3vl_decode_static_scratch_bytes.restype = ctypes.c_size_t
    return L.q3vl_decode_static_scratch_bytes()


def alloc_decode_workspace(model: DeviceTextModel, device="cuda"):
    """Zero-filled device workspace sized for decode_step on this model."""
    import torch
    return torch.zeros(decode_workspace_bytes(model), dtype=torch.uint8, device=device)
