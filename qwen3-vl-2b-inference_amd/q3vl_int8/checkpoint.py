"""The reference's single-file checkpoint: header, text-tensor layout, a writer
and the device loader.

File format (written by export_bin/export_qwen_bin.py:378-420, read by
model/src/load_model.cpp:50-246): a 100-byte little-endian header of 25
int32 / float32 fields (HEADER_FIELDS), then one group per tensor in
TEXT_TENSORS order and then VISION_TENSORS order. An int8 group is its fp32
scales followed by its int8 values (export_qwen_bin.py:346-357 writes a
group's scales before its weights; load_model.cpp:161-163 maps them in that
order); fp16 / fp32 groups are their raw values. Layer-stacked tensors hold
all layers of one sub-key back to back (export_qwen_bin.py:113-119).

The device side is the C ABI: q3vl_checkpoint_load copies the text tensors
into one device allocation and fills a q3vl_text_model for q3vl_decode_step;
q3vl_quantize_groupwise is the exporter's quantizer on the device. The host
helpers here (header packing, the group walk, the writer) move bytes only.
"""
from __future__ import annotations

import ctypes
import struct

import numpy as np

from . import _check, _stream, lib, quantize_groupwise
from .model import DeviceTextModel, TextModelC

_vp = ctypes.c_void_p
_sz = ctypes.c_size_t

# export_qwen_bin.py:36-60 (KEYS) followed by the four quantization fields
# written at :395-401; load_model.cpp:62-91 reads them in this order.
HEADER_FIELDS = [
    ("vocab", "i"), ("hidden", "i"), ("intermediate", "i"), ("layers", "i"), ("heads", "i"),
    ("kv_heads", "i"), ("max_position", "i"), ("rope_theta", "i"), ("rms_eps", "f"),
    ("vision_hidden", "i"), ("vision_depth", "i"), ("vision_patch", "i"),
    ("vision_spatial_merge", "i"), ("vision_temporal_patch", "i"), ("vision_heads", "i"),
    ("vision_intermediate", "i"), ("out_hidden", "i"), ("image_token_id", "i"),
    ("vision_start_token_id", "i"), ("vision_end_token_id", "i"), ("video_token_id", "i"),
    ("text_bits", "i"), ("group_size", "i"), ("vision_bits", "i"), ("group_quantized", "i"),
]
HEADER_BYTES = 100

# File order of the text groups (q3vl_checkpoint_tensor; load_model.cpp:183-195).
# attn_norm is the layers' input_layernorm, read before attention
# (forward.cpp:494); mlp_norm is post_attention_layernorm (forward.cpp:612).
TEXT_TENSORS = ["embed", "attn_norm", "down", "gate", "up", "mlp_norm", "k_norm", "k", "o",
                "q_norm", "q", "v", "final_norm"]
NORM_TENSORS = {"attn_norm", "mlp_norm", "k_norm", "q_norm", "final_norm"}

# Vision groups in file order (load_model.cpp:198-244); the loader fixes 3
# channels, 2304 position embeddings and 3 deep-stack mergers (:104-107).
VISION_TENSORS = [
    "patch_emb_b", "patch_emb_w", "pos_emb_w", "attn_proj_b", "attn_proj_w", "attn_qkv_b",
    "attn_qkv_w", "mlp1_b", "mlp1_w", "mlp2_b", "mlp2_w", "norm1_b", "norm1_w", "norm2_b",
    "norm2_w", "d_mlp1_b", "d_mlp1_w", "d_mlp2_b", "d_mlp2_w", "d_norm_b", "d_norm_w",
    "merge_mlp1_b", "merge_mlp1_w", "merge_mlp2_b", "merge_mlp2_w", "merge_norm_b",
    "merge_norm_w",
]
VISION_CHANNELS, VISION_POS_EMBEDDINGS, DEEP_STACK = 3, 2304, 3


class HeaderC(ctypes.Structure):
    _fields_ = [(n, ctypes.c_float if f == "f" else ctypes.c_int) for n, f in HEADER_FIELDS]


class SpanC(ctypes.Structure):
    _fields_ = [("scales_offset", _sz), ("scales_count", _sz), ("data_offset", _sz),
                ("data_count", _sz), ("bits", ctypes.c_int), ("group", ctypes.c_int)]


def _declare():
    L = lib()
    if getattr(L, "_ck_declared", False):
        return L
    i = ctypes.c_int
    L.q3vl_checkpoint_read_header.restype = i
    L.q3vl_checkpoint_read_header.argtypes = [ctypes.c_char_p, ctypes.POINTER(HeaderC)]
    L.q3vl_checkpoint_text_layout.restype = i
    L.q3vl_checkpoint_text_layout.argtypes = [ctypes.POINTER(HeaderC), ctypes.POINTER(SpanC)]
    L.q3vl_rope_tables.restype = i
    L.q3vl_rope_tables.argtypes = [i, i, i, _vp, _vp]
    L.q3vl_checkpoint_load.restype = i
    L.q3vl_checkpoint_load.argtypes = [ctypes.c_char_p, i, _vp, ctypes.POINTER(_vp)]
    L.q3vl_checkpoint_text_model.restype = ctypes.POINTER(TextModelC)
    L.q3vl_checkpoint_text_model.argtypes = [_vp]
    L.q3vl_checkpoint_header_of.restype = i
    L.q3vl_checkpoint_header_of.argtypes = [_vp, ctypes.POINTER(HeaderC)]
    L.q3vl_checkpoint_free.restype = None
    L.q3vl_checkpoint_free.argtypes = [_vp]
    L._ck_declared = True
    return L


# ------------------------------------------------------------------- header
def pack_header(hdr: dict) -> bytes:
    """The 100 header bytes of a checkpoint (every HEADER_FIELDS key needed)."""
    return b"".join(struct.pack("<" + f, hdr[n]) for n, f in HEADER_FIELDS)


def _to_c(hdr: dict) -> HeaderC:
    c = HeaderC()
    for n, _ in HEADER_FIELDS:
        setattr(c, n, hdr[n])
    return c


def _from_c(c: HeaderC) -> dict:
    return {n: getattr(c, n) for n, _ in HEADER_FIELDS}


def read_header(path: str) -> dict:
    """The header of a checkpoint file, read by the library."""
    L = _declare()
    c = HeaderC()
    _check(L.q3vl_checkpoint_read_header(path.encode(), ctypes.byref(c)))
    return _from_c(c)


def text_layout(hdr: dict) -> dict:
    """name -> span dict (scales_offset, scales_count, data_offset, data_count,
    bits, group) of every text group, as the library walks the file."""
    L = _declare()
    spans = (SpanC * len(TEXT_TENSORS))()
    _check(L.q3vl_checkpoint_text_layout(ctypes.byref(_to_c(hdr)), spans))
    return {n: {f: getattr(spans[i], f) for f, _ in SpanC._fields_}
            for i, n in enumerate(TEXT_TENSORS)}


def rope_tables(rope_theta: int, head_dim: int, rows: int):
    """(cos, sin) fp32 [rows, head_dim/2] text RoPE tables from the library."""
    L = _declare()
    half = head_dim // 2
    cos = np.empty((rows, half), np.float32)
    sin = np.empty((rows, half), np.float32)
    _check(L.q3vl_rope_tables(rope_theta, head_dim, rows, cos.ctypes.data, sin.ctypes.data))
    return cos, sin


# ------------------------------------------------------------------- shapes
def text_shapes(hdr: dict) -> dict:
    """name -> tensor shape of the text groups (load_model.cpp:183-195)."""
    V, H, I, L = hdr["vocab"], hdr["hidden"], hdr["intermediate"], hdr["layers"]
    hd = H // hdr["heads"]
    QD, KV = hdr["heads"] * hd, hdr["kv_heads"] * hd
    return {"embed": (V, H), "attn_norm": (L, H), "down": (L, H, I), "gate": (L, I, H),
            "up": (L, I, H), "mlp_norm": (L, H), "k_norm": (L, hd), "k": (L, KV, H),
            "o": (L, H, H), "q_norm": (L, hd), "q": (L, QD, H), "v": (L, KV, H),
            "final_norm": (H,)}


def vision_shapes(hdr: dict) -> dict:
    """name -> tensor shape of the vision groups (load_model.cpp:198-244)."""
    VH, VD, VP = hdr["vision_hidden"], hdr["vision_depth"], hdr["vision_patch"]
    VTP, VI, OH = hdr["vision_temporal_patch"], hdr["vision_intermediate"], hdr["out_hidden"]
    C, P, D = VISION_CHANNELS, VISION_POS_EMBEDDINGS, DEEP_STACK
    return {
        "patch_emb_b": (VH,), "patch_emb_w": (VH, C, VTP, VP, VP), "pos_emb_w": (P, VH),
        "attn_proj_b": (VD, VH), "attn_proj_w": (VD, VH, VH), "attn_qkv_b": (VD, 3, VH),
        "attn_qkv_w": (VD, 3, VH, VH), "mlp1_b": (VD, VI), "mlp1_w": (VD, VI, VH),
        "mlp2_b": (VD, VH), "mlp2_w": (VD, VH, VI), "norm1_b": (VD, VH), "norm1_w": (VD, VH),
        "norm2_b": (VD, VH), "norm2_w": (VD, VH),
        "d_mlp1_b": (D, VI), "d_mlp1_w": (D, VI, VI), "d_mlp2_b": (D, OH),
        "d_mlp2_w": (D, OH, VI), "d_norm_b": (D, VI), "d_norm_w": (D, VI),
        "merge_mlp1_b": (VI,), "merge_mlp1_w": (VI, VI), "merge_mlp2_b": (OH,),
        "merge_mlp2_w": (OH, VI), "merge_norm_b": (VH,), "merge_norm_w": (VH,),
    }


def quant_group(hdr: dict, name: str) -> int:
    """Values per scale of an int8 text group: group_size when the file is
    group quantized or the tensor is a norm, else the row length
    (export_qwen_bin.py:325-328, load_model.cpp:157-158)."""
    if hdr["group_quantized"] or name in NORM_TENSORS:
        return hdr["group_size"]
    return text_shapes(hdr)[name][-1]


def _raw(arr, bits: int) -> bytes:
    dt = {32: np.float32, 16: np.float16}.get(bits)
    if dt is None:
        raise ValueError(f"{bits}-bit groups are stored raw only as 16 or 32 bits")
    return np.ascontiguousarray(arr, dtype=dt).tobytes()


# ------------------------------------------------------------------- writer
def write_checkpoint(path: str, hdr: dict, text: dict, vision: dict | None = None):
    """Writes a checkpoint in the reference layout.

    text: name -> (q int8, scales fp32) for text_bits 8, or name -> values for
    text_bits 16 / 32. vision: name -> values (vision_bits 16 / 32); missing
    or None -> zeros of the loader's shapes. Shapes are checked against
    text_shapes / vision_shapes."""
    tb, vb = hdr["text_bits"], hdr["vision_bits"]
    ts, vs = text_shapes(hdr), vision_shapes(hdr)
    with open(path, "wb") as f:
        f.write(pack_header(hdr))
        for n in TEXT_TENSORS:
            count = int(np.prod(ts[n]))
            if tb == 8:
                q, s = text[n]
                q = np.ascontiguousarray(q, dtype=np.int8).reshape(-1)
                s = np.ascontiguousarray(s, dtype=np.float32).reshape(-1)
                if q.size != count or s.size != count // quant_group(hdr, n):
                    raise ValueError(f"{n}: {q.size} values / {s.size} scales, expected "
                                     f"{count} / {count // quant_group(hdr, n)}")
                f.write(s.tobytes())
                f.write(q.tobytes())
            else:
                a = np.asarray(text[n])
                if a.size != count:
                    raise ValueError(f"{n}: {a.size} values, expected {count}")
                f.write(_raw(a, tb))
        for n in VISION_TENSORS:
            a = (vision or {}).get(n)
            if a is None:
                a = np.zeros(vs[n], np.float32)
            if np.asarray(a).size != int(np.prod(vs[n])):
                raise ValueError(f"{n}: {np.asarray(a).size} values, expected {vs[n]}")
            f.write(_raw(a, vb))


def export_checkpoint(path: str, hdr: dict, text: dict, vision: dict | None = None,
                      device="cuda"):
    """Quantizes float text tensors with the device quantizer
    (q3vl_quantize_groupwise) and writes the checkpoint: the int8 branch of
    write_weights_streaming (export_qwen_bin.py:297-357). text: name -> fp32
    array or tensor of text_shapes(hdr)[name]."""
    import torch
    if hdr["text_bits"] != 8:  # raw values: no quantization to run
        host = {n: (text[n].detach().cpu().numpy() if isinstance(text[n], torch.Tensor)
                    else np.asarray(text[n])) for n in TEXT_TENSORS}
        write_checkpoint(path, hdr, host, vision)
        return
    packed = {}
    for n in TEXT_TENSORS:
        x = torch.as_tensor(text[n], dtype=torch.float32).to(device).contiguous()
        q, s = quantize_groupwise(x, quant_group(hdr, n))
        packed[n] = (q.cpu().numpy(), s.cpu().numpy())
    write_checkpoint(path, hdr, packed, vision)


# ------------------------------------------------------------------- loader
class Checkpoint:
    """A checkpoint's text model resident on the current device
    (q3vl_checkpoint_load). `model` is a DeviceTextModel for decode_step;
    close() (or the context manager) frees the device memory."""

    def __init__(self, path: str, max_seq: int, stream=None):
        L = _declare()
        h = _vp()
        _check(L.q3vl_checkpoint_load(path.encode(), int(max_seq), _stream(stream),
                                      ctypes.byref(h)))
        self._h = h
        c = HeaderC()
        _check(L.q3vl_checkpoint_header_of(h, ctypes.byref(c)))
        self.header = _from_c(c)
        m = L.q3vl_checkpoint_text_model(h).contents
        model = DeviceTextModel.__new__(DeviceTextModel)
        model.c = TextModelC.from_buffer_copy(m)
        model.dims = {n: getattr(model.c, n) for n in ("vocab", "hidden", "inter", "layers",
                                                       "heads", "kv_heads", "head_dim",
                                                       "max_seq", "gs", "eps")}
        model.t = {}
        self.model = model

    def close(self):
        if self._h:
            _declare().q3vl_checkpoint_free(self._h)
            self._h = None
            self.model = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
