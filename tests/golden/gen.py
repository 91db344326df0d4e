"""Deterministic synthetic inputs shared by the golden-vector writer, the tests
and bench.py (numpy PCG64; shapes and distributions of the BASELINE configs):
W int8 uniform on [-127, 127], S fp32 U(0.001, 0.02) per group, A fp32 N(0,1).
"""
from __future__ import annotations

import hashlib

import numpy as np


def make_case(seed: int, M: int, N: int, K: int, gs: int):
    rng = np.random.default_rng(seed)
    A = rng.standard_normal((M, K), dtype=np.float32)
    W = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    S = rng.uniform(0.001, 0.02, size=(N, K // gs)).astype(np.float32)
    return A, W, S


def sha256(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def tie_group_row(orc, gs: int = 64, K: int = 1024):
    """An activation row whose first group quantizes with a_s == 1.0 exactly,
    so that q = round-half-even(x) on half-integer inputs (0.5 -> 0, 1.5 -> 2,
    2.5 -> 2, ...). Found by search with the oracle; deterministic."""
    ties = np.array([0.5, 1.5, 2.5, 3.5, -0.5, -1.5, -2.5, -3.5], np.float32)
    rng = np.random.default_rng(1234)
    for _ in range(20000):
        small = rng.choice(ties, size=gs - 1)
        rest = 1032256.0 - float(np.sum(small.astype(np.float64) ** 2))
        for delta in range(-40, 41):
            big = np.float32(np.sqrt(rest) + delta * 2e-6)
            row = np.zeros((1, K), np.float32)
            row[0, 0] = big
            row[0, 1:gs] = small
            row[0, gs:] = rng.standard_normal(K - gs).astype(np.float32)
            q, s = orc.quantize_rows(row, gs)
            if s[0, 0] == np.float32(1.0):
                return row
    raise RuntimeError("no tie row found")


# ---------------------------------------------------------------- text model
QWEN3VL_2B = dict(vocab=151936, hidden=2048, inter=6144, layers=28, heads=16, kv_heads=8,
                  head_dim=128, max_seq=3072, gs=64, eps=1e-6, theta=5000000.0)
# hidden = heads * head_dim (forward_text derives head_dim = hidden / heads,
# model/src/forward.cpp:462); every linear dimension >= 1024 keeps each
# projection on the reference's M=1 lane path, as in the full model.
SMALL = dict(vocab=4096, hidden=2048, inter=2048, layers=2, heads=16, kv_heads=8, head_dim=128,
             max_seq=256, gs=64, eps=1e-6, theta=5000000.0)

MODEL_FIELDS = ["emb", "fnorm", "anorm", "mnorm", "qnorm", "knorm"]
LINEARS = ["q", "k", "v", "o", "g", "u", "d"]


def quantize_groupwise(x: np.ndarray, gs: int):
    """The exporter's int8 group quantizer (export_bin/export_qwen_bin.py:260-275):
    per group of gs, scale = (max|x| + 1e-8)/127, q = clip(round_half_even(x/scale))."""
    g = x.reshape(-1, gs).astype(np.float32)
    scale = (np.abs(g).max(axis=1) + np.float32(1e-8)) / np.float32(127.0)
    q = np.clip(np.round(g / scale[:, None]), -127, 127).astype(np.int8)
    return q.reshape(x.shape), scale.astype(np.float32)


def rope_tables(max_seq: int, head_dim: int, theta: float):
    """Text RoPE tables as model/src/load_model.cpp:413-490 builds them (plane
    0, 1-D positions): cos/sin(pos * theta^(-2i/hd)), fp32 [max_seq, hd/2]."""
    i = np.arange(head_dim // 2, dtype=np.float32)
    inv = (np.float32(1.0) / np.power(np.float32(theta), (np.float32(2.0) * i) / np.float32(head_dim),
                                      dtype=np.float32)).astype(np.float32)
    freq = (np.arange(max_seq, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float32)
    return np.cos(freq).astype(np.float32), np.sin(freq).astype(np.float32)


def make_text_model(seed: int, dims: dict):
    """Random-init int8 text decoder of the given dims: linear weights int8
    U[-127,127] with U(0.001,0.02) group scales (as config 0); RMSNorm weights
    U(0.9,1.1) quantized with the exporter's group quantizer."""
    rng = np.random.default_rng(seed)
    V, H, I, L = dims["vocab"], dims["hidden"], dims["inter"], dims["layers"]
    NH, NKV, D, gs = dims["heads"], dims["kv_heads"], dims["head_dim"], dims["gs"]
    m = {}

    def lin(name, N, K, layers=L):
        m["w" + name] = rng.integers(-127, 128, size=(layers, N, K), dtype=np.int8)
        m["s" + name] = rng.uniform(0.001, 0.02, size=(layers, N, K // gs)).astype(np.float32)

    m["emb_w"] = rng.integers(-127, 128, size=(V, H), dtype=np.int8)
    m["emb_s"] = rng.uniform(0.001, 0.02, size=(V, H // gs)).astype(np.float32)
    for name, shape in [("fnorm", (H,)), ("anorm", (L, H)), ("mnorm", (L, H)),
                        ("qnorm", (L, D)), ("knorm", (L, D))]:
        w = rng.uniform(0.9, 1.1, size=shape).astype(np.float32)
        q, s = quantize_groupwise(w, gs)
        m[name + "_w"], m[name + "_s"] = q, s.reshape(shape[:-1] + (shape[-1] // gs,))
    lin("q", NH * D, H)
    lin("k", NKV * D, H)
    lin("v", NKV * D, H)
    lin("o", H, NH * D)
    lin("g", I, H)
    lin("u", I, H)
    lin("d", H, I)
    m["rope_cos"], m["rope_sin"] = rope_tables(dims["max_seq"], D, dims["theta"])
    return m


def make_kv_cache(seed: int, dims: dict, ctx: int):
    """fp16 caches [L, kv_heads, max_seq, hd] holding N(0,1) at positions < ctx."""
    rng = np.random.default_rng(seed)
    shape = (dims["layers"], dims["kv_heads"], dims["max_seq"], dims["head_dim"])
    k = np.zeros(shape, np.float16)
    v = np.zeros(shape, np.float16)
    k[:, :, :ctx] = rng.standard_normal((shape[0], shape[1], ctx, shape[3])).astype(np.float16)
    v[:, :, :ctx] = rng.standard_normal((shape[0], shape[1], ctx, shape[3])).astype(np.float16)
    return k, v
