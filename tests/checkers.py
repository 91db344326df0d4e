"""ctypes wrappers of the CPU checkers (test infrastructure only).

Oracle    -- oracle/liboracle.so, the scalar C restatement of the reference.
Reference -- oracle/_ref/libref_q3vl.so, the reference's own sources compiled
             here (present only where /root/reference was available at build).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
_sz = ctypes.c_size_t
_vp = ctypes.c_void_p


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _build_oracle():
    subprocess.run(["make", "-s", "-C", ORACLE_DIR, "oracle"], check=True)


class Oracle:
    def __init__(self, lib):
        self.lib = lib
        L = lib
        L.orc_quantize_rows.argtypes = [_vp, _sz, _sz, _sz, _vp, _vp]
        L.orc_gemv_lanes.argtypes = [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz]
        L.orc_linear_general.argtypes = [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, ctypes.c_int]
        L.orc_uses_lane_path.argtypes = [_sz, _sz, _sz]
        L.orc_uses_lane_path.restype = ctypes.c_int
        L.orc_linear_i8.argtypes = [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz]
        L.orc_swiglu.argtypes = [_vp, _vp, _sz]
        L.orc_argmax.argtypes = [_vp, _sz]
        L.orc_argmax.restype = ctypes.c_int32
        L.orc_argmax_rows.argtypes = [_vp, _sz, _sz, _vp]

    @classmethod
    def load(cls):
        path = os.path.join(ORACLE_DIR, "liboracle.so")
        if not os.path.exists(path):
            _build_oracle()
        return cls(ctypes.CDLL(path))

    def quantize_rows(self, A, gs):
        A = np.ascontiguousarray(A, np.float32)
        M, K = A.shape
        q = np.zeros((M, K), np.int16)
        s = np.zeros((M, K // gs), np.float32)
        self.lib.orc_quantize_rows(_p(A), M, K, gs, _p(q), _p(s))
        return q, s

    def linear(self, A, W, S, gs, groups=False, path="dispatch"):
        A = np.ascontiguousarray(A, np.float32)
        W = np.ascontiguousarray(W, np.int8)
        S = np.ascontiguousarray(S, np.float32)
        M, K = A.shape
        N = W.shape[0]
        C = np.zeros((M, N), np.float32)
        G = np.zeros((M, N, K // gs), np.int32) if groups else None
        if path == "dispatch":
            self.lib.orc_linear_i8(_p(A), _p(W), _p(S), _p(C), _p(G), M, N, K, gs)
        elif path == "lanes":
            self.lib.orc_gemv_lanes(_p(A), _p(W), _p(S), _p(C), _p(G), N, K, gs)
        else:
            self.lib.orc_linear_general(_p(A), _p(W), _p(S), _p(C), _p(G), M, N, K, gs,
                                        0 if path == "general_nofma" else 1)
        return (C, G) if groups else C

    def uses_lane_path(self, M, N, K):
        return bool(self.lib.orc_uses_lane_path(M, N, K))

    def swiglu(self, gate, up):
        g = np.array(gate, np.float32, copy=True)
        u = np.ascontiguousarray(up, np.float32)
        self.lib.orc_swiglu(_p(g), _p(u), g.size)
        return g

    # ---- decode step
    def quantize_groupwise(self, x, group):
        """The exporter's group quantizer: (q int8 like x, scales [x.size/group])."""
        L = self.lib
        L.orc_quantize_groupwise.argtypes = [_vp, _sz, _sz, _vp, _vp]
        x = np.ascontiguousarray(x, np.float32)
        q = np.zeros(x.shape, np.int8)
        s = np.zeros(x.size // group, np.float32)
        L.orc_quantize_groupwise(_p(x), x.size, group, _p(q), _p(s))
        return q, s

    def decode_step(self, dims, arrays, k_cache, v_cache, token, pos, kv_fp16=True, chunked=False):
        """Returns (next_id, logits); updates the caches at pos in place.
        chunked: the chunked attention order (Q3VL_ATTN_CHUNKED)."""
        L = self.lib
        L.orc_decode_step.restype = ctypes.c_int32
        L.orc_decode_step.argtypes = [_vp, _vp, _vp, ctypes.c_int, ctypes.c_int32, _sz, _vp]
        st = _model_struct(dims, arrays)
        logits = np.zeros(dims["vocab"], np.float32)
        flags = (1 if kv_fp16 else 0) | (2 if chunked else 0)
        nid = L.orc_decode_step(ctypes.byref(st), _p(k_cache), _p(v_cache), flags, token,
                                pos, _p(logits))
        return int(nid), logits

    def rms_norm_i8(self, x, w, ws, gs, eps):
        L = self.lib
        L.orc_rms_norm_i8.argtypes = [_vp, _vp, _vp, _sz, _sz, ctypes.c_float, _vp]
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros_like(x)
        L.orc_rms_norm_i8(_p(x), _p(w), _p(ws), x.size, gs, eps, _p(out))
        return out

    def rms_norm_inplace_i8(self, x, w, ws, gs, eps, batches):
        L = self.lib
        L.orc_rms_norm_inplace_i8.argtypes = [_vp, _vp, _vp, _sz, _sz, ctypes.c_float, _sz]
        x = np.array(x, np.float32, copy=True)
        L.orc_rms_norm_inplace_i8(_p(x), _p(w), _p(ws), x.size // batches, gs, eps, batches)
        return x

    def rope(self, x, cos_row, sin_row, heads, hd):
        L = self.lib
        L.orc_rope.argtypes = [_vp, _vp, _vp, _sz, _sz]
        x = np.array(x, np.float32, copy=True)
        L.orc_rope(_p(x), _p(np.ascontiguousarray(cos_row)), _p(np.ascontiguousarray(sin_row)),
                   heads, hd)
        return x

    def softmax(self, x):
        L = self.lib
        L.orc_softmax.argtypes = [_vp, _sz]
        x = np.array(x, np.float32, copy=True)
        L.orc_softmax(_p(x), x.size)
        return x

    def attention(self, q, kc, vc, heads, kv_heads, hd, max_seq, pos):
        L = self.lib
        L.orc_attention.argtypes = [_vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _vp, _vp]
        att = np.zeros(pos + 1, np.float32)
        out = np.zeros(heads * hd, np.float32)
        L.orc_attention(_p(np.ascontiguousarray(q, np.float32)), _p(np.ascontiguousarray(kc, np.float32)),
                        _p(np.ascontiguousarray(vc, np.float32)), heads, kv_heads, hd, max_seq, pos,
                        _p(att), _p(out))
        return out

    def attention_chunked(self, q, kc, vc, heads, kv_heads, hd, max_seq, pos):
        """The chunked attention order (Q3VL_ATTN_CHUNKED) of one layer."""
        L = self.lib
        L.orc_attention_chunked.argtypes = [_vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _vp, _vp]
        att = np.zeros(pos + 1, np.float32)
        out = np.zeros(heads * hd, np.float32)
        L.orc_attention_chunked(_p(np.ascontiguousarray(q, np.float32)),
                                _p(np.ascontiguousarray(kc, np.float32)),
                                _p(np.ascontiguousarray(vc, np.float32)), heads, kv_heads, hd,
                                max_seq, pos, _p(att), _p(out))
        return out

    def argmax_rows(self, logits):
        x = np.ascontiguousarray(logits, np.float32)
        if x.ndim == 1:
            x = x[None]
        ids = np.zeros(x.shape[0], np.int32)
        self.lib.orc_argmax_rows(_p(x), x.shape[0], x.shape[1], _p(ids))
        return ids


def _model_struct(dims, arrays):
    """orc_model / ref_model_desc over numpy arrays (same layout as the C ABI's
    q3vl_text_model); keeps the arrays alive on the returned struct."""
    import sys as _sys
    pkg = os.path.join(ROOT, "qwen3-vl-2b-inference_amd")
    if pkg not in _sys.path:
        _sys.path.insert(0, pkg)
    from q3vl_int8.model import make_struct
    arrs = {k: np.ascontiguousarray(v) for k, v in arrays.items()}
    st = make_struct(dims, lambda n: arrs[n].ctypes.data)
    st._keep = arrs
    return st


class _RefCkTensor(ctypes.Structure):
    _fields_ = [("data", _vp), ("scales", _vp), ("count", _sz), ("group", _sz),
                ("dtype", ctypes.c_int)]


class Reference:
    def __init__(self, lib):
        self.lib = lib
        lib.ref_linear_i8.argtypes = [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz]
        lib.ref_swiglu.argtypes = [_vp, _vp, _sz]

    @classmethod
    def load(cls):
        path = os.path.join(ORACLE_DIR, "_ref", "libref_q3vl.so")
        if not os.path.exists(path):
            return None
        return cls(ctypes.CDLL(path))

    def linear(self, A, W, S, gs):
        A = np.ascontiguousarray(A, np.float32)
        W = np.ascontiguousarray(W, np.int8)
        S = np.ascontiguousarray(S, np.float32)
        M, K = A.shape
        N = W.shape[0]
        C = np.zeros((M, N), np.float32)
        self.lib.ref_linear_i8(_p(A), _p(W), _p(S), _p(C), M, N, K, gs)
        return C

    def swiglu(self, gate, up):
        g = np.array(gate, np.float32, copy=True)
        u = np.ascontiguousarray(up, np.float32)
        self.lib.ref_swiglu(_p(g), _p(u), g.size)
        return g

    def checkpoint_open(self, path):
        """The reference loader over a checkpoint file: (header fields in file
        order with rms_eps as a float, [tensor dicts] for the 13 text then 27
        vision groups, close())."""
        L = self.lib
        L.ref_checkpoint_open.restype = _vp
        L.ref_checkpoint_open.argtypes = [ctypes.c_char_p, _vp, _vp]
        L.ref_checkpoint_close.argtypes = [_vp]
        cfg = np.zeros(25, np.int32)
        ts = (_RefCkTensor * 40)()
        h = L.ref_checkpoint_open(path.encode(), _p(cfg), ts)
        if not h:
            raise RuntimeError(f"reference loader mapped nothing from {path}")
        fields = [int(v) for v in cfg]
        fields[8] = float(cfg[8:9].view(np.float32)[0])
        out = [dict(data=t.data, scales=t.scales, count=t.count, group=t.group, dtype=t.dtype)
               for t in ts]
        return fields, out, (lambda: L.ref_checkpoint_close(h))

    def rope_precompute(self, rope_theta, hidden, heads, seq_len):
        """qwen_rope_precompute's (cos, sin) [3, seq_len, head_dim/2]."""
        L = self.lib
        L.ref_rope_precompute.argtypes = [ctypes.c_int] * 4 + [_vp, _vp]
        half = hidden // heads // 2
        cos = np.zeros((3, seq_len, half), np.float32)
        sin = np.zeros((3, seq_len, half), np.float32)
        L.ref_rope_precompute(rope_theta, hidden, heads, seq_len, _p(cos), _p(sin))
        return cos, sin

    def rms_norm_i8(self, x, w, ws, gs, eps):
        L = self.lib
        L.ref_rms_norm_i8.argtypes = [_vp, _vp, _vp, _sz, _sz, ctypes.c_float, _vp]
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros_like(x)
        L.ref_rms_norm_i8(_p(x), _p(w), _p(ws), x.size, gs, eps, _p(out))
        return out

    def rms_norm_inplace_i8(self, x, w, ws, gs, eps, batches):
        L = self.lib
        L.ref_rms_norm_inplace_i8.argtypes = [_vp, _vp, _vp, _sz, _sz, ctypes.c_float, _sz]
        x = np.array(x, np.float32, copy=True)
        L.ref_rms_norm_inplace_i8(_p(x), _p(w), _p(ws), x.size // batches, gs, eps, batches)
        return x

    def rope(self, x, cos_t, sin_t, heads, hd, pos):
        L = self.lib
        L.ref_rope.argtypes = [_vp, _vp, _vp, _sz, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        x = np.array(x, np.float32, copy=True)
        L.ref_rope(_p(x), _p(np.ascontiguousarray(cos_t)), _p(np.ascontiguousarray(sin_t)),
                   cos_t.shape[0], heads, hd, pos)
        return x

    def softmax(self, x):
        L = self.lib
        L.ref_softmax.argtypes = [_vp, _sz]
        x = np.array(x, np.float32, copy=True)
        L.ref_softmax(_p(x), x.size)
        return x

    def attention(self, q, kc, vc, heads, kv_heads, hd, max_seq, pos):
        L = self.lib
        L.ref_attention.argtypes = [_vp, _vp, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, _sz,
                                    ctypes.c_int, _vp]
        out = np.zeros(heads * hd, np.float32)
        L.ref_attention(_p(np.ascontiguousarray(q, np.float32)), _p(np.ascontiguousarray(kc, np.float32)),
                        _p(np.ascontiguousarray(vc, np.float32)), heads, kv_heads, hd, max_seq, pos,
                        _p(out))
        return out

    def decoder(self, dims, arrays, k_cache32, v_cache32):
        """The reference's forward_text over fp32 caches (updated in place)."""
        L = self.lib
        L.ref_decoder_create.restype = _vp
        L.ref_decoder_create.argtypes = [_vp, _vp, _vp]
        L.ref_decoder_step.restype = ctypes.c_int
        L.ref_decoder_step.argtypes = [_vp, ctypes.c_int, _sz, _vp]
        L.ref_decoder_destroy.argtypes = [_vp]
        st = _model_struct(dims, arrays)
        h = L.ref_decoder_create(ctypes.byref(st), _p(k_cache32), _p(v_cache32))
        ref = self

        class _Dec:
            max_seq = int(dims["max_seq"])

            def step(self_, token, pos):
                """Logits of forward_text at pos; ValueError (and no call) when
                pos >= max_seq or the token is outside the vocabulary."""
                logits = np.zeros(dims["vocab"], np.float32)
                if L.ref_decoder_step(h, int(token), int(pos), _p(logits)) != 0:
                    raise ValueError(f"reference decode step refused: token {token}, pos {pos}, "
                                     f"max_seq {dims['max_seq']}, vocab {dims['vocab']}")
                return logits

            def close(self_):
                L.ref_decoder_destroy(h)

        d = _Dec()
        d._keep = (st, k_cache32, v_cache32, ref)
        return d
