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

    def argmax_rows(self, logits):
        x = np.ascontiguousarray(logits, np.float32)
        if x.ndim == 1:
            x = x[None]
        ids = np.zeros(x.shape[0], np.int32)
        self.lib.orc_argmax_rows(_p(x), x.shape[0], x.shape[1], _p(ids))
        return ids


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
