#!/usr/bin/env python3
"""Benchmark of the MI355X int8 group-quantized matmul path.

Prints ONE JSON line (rank 0, N=1). Workloads are BASELINE.json's configs on
synthetic seeded inputs (tests/golden/gen.py distributions: int8 U[-127,127]
weights, U(0.001,0.02) group scales, N(0,1) activations), weights resident in
HBM before any timed region.

Headline (config 1): greedy decode of the full Qwen3-VL-2B text decoder (28
layers, hidden 2048, 16/8 heads of 128, intermediate 6144, vocab 151936,
int8 weights with group-64 scales, fp16 KV cache prefilled with N(0,1) at
context 1024, batch 1). One step = one token: q3vl_decode_step captured once
in a HIP graph and replayed; token and position live in device memory and
each replay writes the next token and advances the position, so K steps
generate K tokens at contexts 1024+W .. 1024+W+K-1. value = tokens/s.

roofline: the dominant kernel of the decode step, gemv_kernel (every linear
of the step and the lm_head; M=1 lane path), at the decode step's shapes:
achieved = algorithmic bytes (int8 weights + fp32 group scales + fp32
activations in and out) summed over one step's GEMV launches / the summed
kernel durations, measured as HIP-graph replays of each class of launch
between HIP events on the replaying stream; peak = 8 TB/s HBM.

cpu_baseline: the reference's own forward_text (oracle/_ref, compiled from the
reference sources; fp32 KV cache as the reference keeps it) on the same model
and context, timed on this host's cores for a bounded number of tokens.

Also reported under "configs": config 0 (up_proj GEMV, GB/s), config 2
(prefill gate|up+SwiGLU and down at M=512, TOPS), config 3 (lm_head GEMV +
argmax, M=1 and 8, GB/s), config 4 (vision-encoder linears, TOPS), the
exporter's weight quantizer on one up_proj ("export", GB/s) and, with
--configs ...,load, the load of a full-size checkpoint file into HBM (GB/s of
file bytes, page-cache-resident file).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "qwen3-vl-2b-inference_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0   # dense int8 MFMA
# The GEMMs run on fp16 MFMA: exact fp16 images of the int16 activations and
# int8 weights (every product and every in-group sum is exact in fp32), so the
# unit's dense fp16 peak bounds them; the int8 fraction is reported beside it.
FP16_PEAK_TFLOPS = 2500.0
GS = 64
CTX = 1024


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _event_time(fn, steps, warmup):
    """ms per call of fn over `steps` calls, HIP events on the current stream."""
    import torch
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for i in range(steps):
        fn(warmup + i)
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def _graph_time(fns, reps=5, trials=5):
    """ms per call of the calls in fns, captured once into a HIP graph and
    replayed (median of `trials` timings of `reps` replays): the kernels'
    own time, without the per-call host overhead of eager launches."""
    import torch
    for fn in fns:  # eager pass: first use
        fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for fn in fns:
            fn()
    g.replay()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    out = []
    for _ in range(trials):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        for _ in range(reps):
            g.replay()
        e1.record(st)
        torch.cuda.synchronize()
        out.append(e0.elapsed_time(e1) / (reps * len(fns)))
    return sorted(out)[len(out) // 2]


def gen_weights(N, K, copies, seed, device="cuda"):
    """int8 weights U[-127,127] and U(0.001, 0.02) group scales, generated on
    the device from a seeded generator."""
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    Ws, Ss = [], []
    for _ in range(copies):
        Ws.append(torch.randint(-127, 128, (N, K), dtype=torch.int8, device=device, generator=g))
        Ss.append(torch.rand((N, K // GS), dtype=torch.float32, device=device, generator=g)
                  * 0.019 + 0.001)
    return Ws, Ss


def copies_for(bytes_per_copy, floor=2):
    """Distinct weight copies so the rotating working set exceeds 2x the
    256 MB Infinity Cache."""
    return max(floor, int((600 << 20) // bytes_per_copy) + 1)


def wbytes(N, K):
    return N * K + N * (K // GS) * 4


# ------------------------------------------------------------------ config 1
def decode_dims(max_seq):
    from golden.gen import QWEN3VL_2B
    return dict(QWEN3VL_2B, max_seq=max_seq)


def build_model(dims, seed):
    from golden.gen import make_kv_cache, make_text_model
    t = time.perf_counter()
    m = make_text_model(seed, dims)
    k16, v16 = make_kv_cache(seed + 1, dims, CTX)
    log(f"bench: model + caches generated in {time.perf_counter() - t:.1f} s")
    return m, k16, v16


def bench_cfg1(args, m, k16, v16, dims):
    import torch
    from q3vl_int8 import model as qm
    model = qm.DeviceTextModel(dims, m)
    kd = torch.from_numpy(k16.view("int16")).cuda()
    vd = torch.from_numpy(v16.view("int16")).cuda()
    tok = torch.tensor([dims["vocab"] - 936], dtype=torch.int32, device="cuda")
    pos = torch.tensor([CTX], dtype=torch.int32, device="cuda")
    logits = torch.empty(dims["vocab"], dtype=torch.float32, device="cuda")
    ws = qm.alloc_decode_workspace(model)

    def step():
        qm.decode_step(model, kd, vd, tok, pos, logits, ws)

    # eager steps (first use of every kernel), then back to context CTX
    step()
    step()
    torch.cuda.synchronize()
    eager_ms = _event_time(lambda i: step(), 10, 0)
    pos.fill_(CTX)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    torch.cuda.synchronize()
    pos.fill_(CTX)
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        g.replay()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(args.steps):
        g.replay()
    e1.record(st)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    end_pos = int(pos.item())
    assert end_pos == CTX + args.warmup + args.steps, (end_pos, args.warmup, args.steps)
    step_bytes = decode_step_weight_bytes(dims)
    res = dict(name="cfg1_decode_step", metric="tok/s", value=1000.0 / ms, ms=ms,
               eager_ms=eager_ms, contexts=[CTX + args.warmup, end_pos - 1],
               weight_bytes_per_token=step_bytes,
               effective_weight_GBs=step_bytes / (ms * 1e-3) / 1e9)
    res["gemv_roofline"] = decode_gemv_roofline(model, dims)
    return res


def decode_gemv_shapes(dims):
    """(name, segments [(N, K)], activation K, outputs N, extra bytes) per
    GEMV launch of one decode step, as q3vl_decode_step issues them."""
    H, I, V = dims["hidden"], dims["inter"], dims["vocab"]
    QD, KD = dims["heads"] * dims["head_dim"], dims["kv_heads"] * dims["head_dim"]
    per_layer = [("qkv", [(QD, H), (KD, H), (KD, H)]), ("o", [(H, QD)]),
                 ("gate_up", [(I, H), (I, H)]), ("down", [(H, I)])]
    return per_layer, ("lm_head", [(V, H)])


def decode_step_weight_bytes(dims):
    per_layer, head = decode_gemv_shapes(dims)
    b = sum(wbytes(N, K) for _, segs in per_layer for N, K in segs) * dims["layers"]
    return b + sum(wbytes(N, K) for N, K in head[1])


def decode_gemv_roofline(model, dims):
    """Every GEMV launch of one decode step at its shape, with its layer's
    weights (the lm_head in plain mode). Each class of launch (qkv, o,
    gate/up, down over the 28 layers; lm_head four times) is captured in a
    HIP graph and replayed between HIP events on the capturing stream, so
    launch gaps vanish and time / launches is the average kernel duration
    (median of five timed trials).
    achieved = one step's algorithmic bytes / one step's summed durations."""
    import torch
    import q3vl_int8 as q
    t = model.t
    H, I, V, L = dims["hidden"], dims["inter"], dims["vocab"], dims["layers"]
    QD, KD = dims["heads"] * dims["head_dim"], dims["kv_heads"] * dims["head_dim"]
    x = torch.randn((1, max(H, I, QD)), dtype=torch.float32, device="cuda")
    xH, xI, xQ = x[:, :H].contiguous(), x[:, :I].contiguous(), x[:, :QD].contiguous()
    outs = {n: torch.empty((1, n), dtype=torch.float32, device="cuda") for n in {QD, KD, H, I, V}}
    kv2 = torch.empty_like(outs[KD])
    ws = q.alloc_workspace(1, V, max(H, I), GS)
    kinds = {
        "qkv": ([lambda l=l: q.linear_i8_multi(xH, [t["wq"][l], t["wk"][l], t["wv"][l]],
                                               [t["sq"][l], t["sk"][l], t["sv"][l]], GS,
                                               outs=[outs[QD], outs[KD], kv2], workspace=ws)
                 for l in range(L)],
                wbytes(QD, H) + 2 * wbytes(KD, H) + H * 4 + (QD + 2 * KD) * 4),
        "o": ([lambda l=l: q.linear_i8(xQ, t["wo"][l], t["so"][l], GS, out=outs[H], workspace=ws)
               for l in range(L)], wbytes(H, QD) + QD * 4 + H * 4),
        "gate_up": ([lambda l=l: q.linear_i8_swiglu(xH, t["wg"][l], t["sg"][l], t["wu"][l],
                                                    t["su"][l], GS, out=outs[I], workspace=ws)
                     for l in range(L)], 2 * wbytes(I, H) + H * 4 + I * 4),
        "down": ([lambda l=l: q.linear_i8(xI, t["wd"][l], t["sd"][l], GS, out=outs[H], workspace=ws)
                  for l in range(L)], wbytes(H, I) + I * 4 + H * 4),
        "lm_head": ([lambda: q.linear_i8(xH, t["emb_w"], t["emb_s"], GS, out=outs[V], workspace=ws)] * 4,
                    wbytes(V, H) + H * 4 + V * 4),
    }
    per_step = {"qkv": L, "o": L, "gate_up": L, "down": L, "lm_head": 1}
    res = {}
    for name, (fns, nbytes) in kinds.items():
        for fn in fns:  # eager pass: first use
            fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for fn in fns:
                fn()
        g.replay()
        torch.cuda.synchronize()
        st = torch.cuda.current_stream()
        reps, trials = 5, []
        for _ in range(5):  # median of 5 timed trials of 5 replays each
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(st)
            for _ in range(reps):
                g.replay()
            e1.record(st)
            torch.cuda.synchronize()
            trials.append(e0.elapsed_time(e1) * 1e3 / (reps * len(fns)))
        us = sorted(trials)[len(trials) // 2]
        res[name] = dict(us=us, bytes=nbytes, GBs=nbytes / (us * 1e-6) / 1e9)
    step_us = sum(res[k]["us"] * n for k, n in per_step.items())
    step_bytes = sum(res[k]["bytes"] * n for k, n in per_step.items())
    launches = sum(per_step.values())
    gbs = step_bytes / (step_us * 1e-6) / 1e9
    return dict(kernel="gemv_kernel<64, 1, true, R> (R = rows per tile: 2, 4 or 8 by shape)", launches=launches,
                bytes_per_launch=step_bytes / launches, avg_launch_us=step_us / launches,
                achieved_GBs=gbs, frac=gbs / HBM_PEAK_GBS, step_gemv_us=step_us, by_class=res)


def cpu_baseline_cfg1(m, k16, v16, dims, budget_s):
    """forward_text of the reference (oracle/_ref) on the same model at the
    same context: tokens for about budget_s seconds, one thread per core the
    OpenMP runtime uses."""
    from checkers import Reference
    ref = Reference.load()
    if ref is None:
        return None
    k32, v32 = k16.astype("float32"), v16.astype("float32")
    dec = ref.decoder(dims, m, k32, v32)
    try:
        tok = dims["vocab"] - 936
        t0 = time.perf_counter()
        lg = dec.step(tok, CTX)
        first = time.perf_counter() - t0
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < budget_s and n < 200:
            tok = int(lg.argmax())
            lg = dec.step(tok, CTX + 1 + n)
            n += 1
        el = time.perf_counter() - t0
    finally:
        dec.close()
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return dict(value=n / el, unit="tok/s", cores=threads, kind="reference",
                sample=f"{n} greedy decode steps of forward_text (28 layers, fp32 KV cache) at "
                       f"contexts {CTX + 1}..{CTX + n}, after one untimed step ({first:.2f} s)")


# ------------------------------------------------------------- configs 0,2,3,4
def bench_cfg0(args):
    import torch
    import q3vl_int8 as q
    N, K = 6144, 2048
    n = copies_for(wbytes(N, K))
    Ws, Ss = gen_weights(N, K, n, 0xC0FFEE00)
    x = torch.randn((1, K), dtype=torch.float32, device="cuda")
    y = torch.empty((1, N), dtype=torch.float32, device="cuda")
    ws = q.alloc_workspace(1, N, K, GS)
    call = lambda i: q.linear_i8(x, Ws[i % n], Ss[i % n], GS, out=y, workspace=ws)
    eager_ms = _event_time(call, max(args.steps, 200), 20)
    # One graph of the n launches (one per weight copy), replayed: a 6 us
    # kernel is shorter than a Python call, so eager calls would time the host
    ms = _graph_time([lambda i=i: call(i) for i in range(n)])
    algo = wbytes(N, K) + K * 4 + N * 4
    gbs = algo / (ms * 1e-3) / 1e9
    return dict(name="cfg0_up_proj_gemv", metric="GB/s", value=gbs, ms=ms, eager_ms=eager_ms,
                algo_bytes=algo, frac=gbs / HBM_PEAK_GBS, copies=n,
                timing="HIP-graph replay of one launch per weight copy (eager_ms: per Python call)",
                kernel="gemv_kernel<64, 1, true, 4>")


def bench_cfg2(args):
    import torch
    import q3vl_int8 as q
    M, K, I = 512, 2048, 6144
    Wg, Sg = gen_weights(I, K, 1, 1)
    Wu, Su = gen_weights(I, K, 1, 2)
    Wd, Sd = gen_weights(K, I, 1, 3)
    A = torch.randn((M, K), dtype=torch.float32, device="cuda")
    H = torch.empty((M, I), dtype=torch.float32, device="cuda")
    D = torch.empty((M, K), dtype=torch.float32, device="cuda")
    ws = q.alloc_workspace(M, I, max(K, I), GS)

    def step(i):
        q.linear_i8_swiglu(A, Wg[0], Sg[0], Wu[0], Su[0], GS, out=H, workspace=ws)
        q.linear_i8(H, Wd[0], Sd[0], GS, out=D, workspace=ws)

    ms = _event_time(step, max(args.steps // 2, 50), 5)
    ops = 2 * M * (2 * I) * K + 2 * M * K * I
    tops = ops / (ms * 1e-3) / 1e12
    return dict(name="cfg2_prefill_gemm", metric="TOPS", value=tops, ms=ms, algo_ops=ops,
                frac=tops / FP16_PEAK_TFLOPS, frac_of_int8_peak=tops / INT8_PEAK_TOPS,
                kernel="quantize_rows_kernel + gemm_g64_kernel<MT, NT, SWIGLU, D>")


def bench_cfg3(args, M):
    import torch
    import q3vl_int8 as q
    V, K = 151936, 2048
    n = 3  # 3 x 330 MB > 2x the Infinity Cache
    Ws, Ss = gen_weights(V, K, n, 0xC0FFEE03)
    x = torch.randn((M, K), dtype=torch.float32, device="cuda")
    ids = torch.empty((M,), dtype=torch.int32, device="cuda")
    ws = q.alloc_workspace(M, V, K, GS)
    # eager: each call keeps the device busy for ~60-190 us, longer than the
    # host needs to issue the next, so no host time is inside the figure
    ms = _event_time(lambda i: q.lm_head_argmax(x, Ws[i % n], Ss[i % n], GS, ids=ids, workspace=ws),
                     max(args.steps // 2, 50), 6)
    algo = wbytes(V, K) + M * K * 4 + M * 4
    gbs = algo / (ms * 1e-3) / 1e9
    return dict(name=f"cfg3_lm_head_argmax_m{M}", metric="GB/s", value=gbs, ms=ms, algo_bytes=algo,
                frac=gbs / HBM_PEAK_GBS)


def bench_cfg4(args):
    """24 ViT blocks (qkv, proj, fc1, fc2 over 784 patch tokens) and the 2x2
    merger projection (196 tokens): every int8 GEMM of the vision encoder
    with its own random weights."""
    import torch
    import q3vl_int8 as q
    T, D, F, B = 784, 1024, 4096, 24
    shapes = [(3 * D, D), (D, D), (F, D), (D, F)]
    Wb = [[gen_weights(N, K, 1, 7000 + 10 * b + j) for j, (N, K) in enumerate(shapes)]
          for b in range(B)]
    Wm, Sm = gen_weights(2048, 4 * D, 1, 7999)
    xD = torch.randn((T, D), dtype=torch.float32, device="cuda")
    xF = torch.randn((T, F), dtype=torch.float32, device="cuda")
    xM = torch.randn((T // 4, 4 * D), dtype=torch.float32, device="cuda")
    outs = {N: torch.empty((T, N), dtype=torch.float32, device="cuda") for N, _ in shapes}
    outM = torch.empty((T // 4, 2048), dtype=torch.float32, device="cuda")
    ws = q.alloc_workspace(T, 3 * D, F, GS)

    def step(i):
        for b in range(B):
            for j, (N, K) in enumerate(shapes):
                (W,), (S,) = Wb[b][j]
                q.linear_i8(xF if K == F else xD, W, S, GS, out=outs[N], workspace=ws)
        q.linear_i8(xM, Wm[0], Sm[0], GS, out=outM, workspace=ws)

    ms = _event_time(step, max(args.steps // 20, 10), 2)
    ops = B * sum(2 * T * N * K for N, K in shapes) + 2 * (T // 4) * 2048 * 4 * D
    tops = ops / (ms * 1e-3) / 1e12
    return dict(name="cfg4_vision_linears", metric="TOPS", value=tops, ms=ms, algo_ops=ops,
                frac=tops / FP16_PEAK_TFLOPS, frac_of_int8_peak=tops / INT8_PEAK_TOPS, gemms=B * 4 + 1,
                kernel="quantize_rows_kernel + gemm_g64_kernel<MT, NT, SWIGLU, D>")


# ------------------------------------------------- checkpoint files
def bench_export(args):
    """q3vl_quantize_groupwise over one up_proj [6144, 2048] fp32 at group 64."""
    import torch
    import q3vl_int8 as q
    N, K = 6144, 2048
    n = copies_for(N * K * 4)
    g = torch.Generator(device="cuda")
    g.manual_seed(0xF4)
    Xs = [torch.randn((N, K), dtype=torch.float32, device="cuda", generator=g) * 0.02
          for _ in range(n)]
    qo = torch.empty((N, K), dtype=torch.int8, device="cuda")
    so = torch.empty((N * K // GS,), dtype=torch.float32, device="cuda")
    ms = _event_time(lambda i: q.quantize_groupwise(Xs[i % n], GS, qo, so),
                     max(args.steps, 200), 20)
    algo = N * K * 4 + N * K + (N * K // GS) * 4
    gbs = algo / (ms * 1e-3) / 1e9
    return dict(name="export_quantizer", metric="GB/s", value=gbs, ms=ms, algo_bytes=algo,
                frac=gbs / HBM_PEAK_GBS, copies=n, kernel="quantize_export_vec_kernel<64, 2>")


def bench_load(args):
    """Loads a full-size (28-layer, vocab 151936, group 64) checkpoint file
    into HBM with q3vl_checkpoint_load; the file is written first (random
    int8 values and U(0.001,0.02) scales), so it is page-cache resident."""
    import tempfile

    import numpy as np
    from q3vl_int8 import checkpoint as ck
    hdr = dict(vocab=151936, hidden=2048, intermediate=6144, layers=28, heads=16, kv_heads=8,
               max_position=262144, rope_theta=5000000, rms_eps=1e-6, vision_hidden=1024,
               vision_depth=24, vision_patch=16, vision_spatial_merge=2,
               vision_temporal_patch=2, vision_heads=16, vision_intermediate=4096,
               out_hidden=2048, image_token_id=151655, vision_start_token_id=151652,
               vision_end_token_id=151653, video_token_id=151656, text_bits=8,
               group_size=GS, vision_bits=16, group_quantized=1)
    spans = ck.text_layout(hdr)
    rng = np.random.default_rng(0xF1)
    pool_q = rng.integers(-127, 128, size=64 << 20, dtype=np.int8).tobytes()
    pool_s = rng.uniform(0.001, 0.02, size=16 << 20).astype(np.float32).tobytes()
    d = tempfile.mkdtemp()
    path = os.path.join(d, "qwen3vl_2b_text_i8.bin")
    try:
        with open(path, "wb") as f:
            f.write(ck.pack_header(hdr))
            for n in ck.TEXT_TENSORS:
                for nbytes, pool in ((spans[n]["scales_count"] * 4, pool_s),
                                     (spans[n]["data_count"], pool_q)):
                    while nbytes:
                        k = min(nbytes, len(pool))
                        f.write(pool[:k])
                        nbytes -= k
        end = spans["final_norm"]["data_offset"] + spans["final_norm"]["data_count"]
        text_bytes = end - ck.HEADER_BYTES
        times = []
        for _ in range(3):
            t = time.perf_counter()
            c = ck.Checkpoint(path, max_seq=4096)
            times.append(time.perf_counter() - t)
            c.close()
        best = min(times)
    finally:
        try:
            os.remove(path)
        finally:
            os.rmdir(d)
    return dict(name="checkpoint_load", metric="GB/s", value=text_bytes / best / 1e9,
                ms=best * 1e3, text_bytes=text_bytes, runs_s=[round(x, 4) for x in times],
                note="file bytes / wall time of q3vl_checkpoint_load (allocation, reads from "
                     "the page cache, host-to-device copies, RoPE tables for 4096 rows)")


def cpu_baseline_cfg0(budget_s):
    """The reference's linear() (oracle/_ref) on config 0's shape."""
    import numpy as np
    from checkers import Reference
    from golden.gen import make_case
    ref = Reference.load()
    if ref is None:
        return None
    N, K = 6144, 2048
    A, W, S = make_case(0xC0FFEE00, 1, N, K, GS)
    ref.linear(A, W, S, GS)
    t0, times = time.perf_counter(), []
    while time.perf_counter() - t0 < budget_s:
        t = time.perf_counter()
        ref.linear(A, W, S, GS)
        times.append(time.perf_counter() - t)
    med = float(np.median(times))
    algo = wbytes(N, K) + K * 4 + N * 4
    return dict(value=algo / med / 1e9, unit="GB/s", cores=int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)),
                kind="reference", sample=f"{len(times)} calls of linear() M=1 N=6144 K=2048, median {med * 1e3:.3f} ms")


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_gemv_traffic.json")


def pmc_workload():
    """Workload for the HBM-traffic counter passes (rocprofv3 --pmc
    FETCH_SIZE, then WRITE_SIZE): an elementwise dst = src + 1 over 256 MiB of
    uint8 (the calibration kernel: 256 MiB read, 256 MiB written) and then 3
    eager decode steps of config 1, whose gemv_kernel dispatches are the
    measured kernel."""
    import torch
    from q3vl_int8 import model as qm
    n = 256 << 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    torch.add(src, 1, out=dst)
    torch.cuda.synchronize()
    dims = decode_dims(max_seq=CTX + 16)
    m, k16, v16 = build_model(dims, 0xD0C0DE)
    model = qm.DeviceTextModel(dims, m)
    kd = torch.from_numpy(k16.view("int16")).cuda()
    vd = torch.from_numpy(v16.view("int16")).cuda()
    tok = torch.tensor([5], dtype=torch.int32, device="cuda")
    pos = torch.tensor([CTX], dtype=torch.int32, device="cuda")
    ws = qm.alloc_decode_workspace(model)
    for _ in range(3):
        qm.decode_step(model, kd, vd, tok, pos, None, ws)
    torch.cuda.synchronize()
    log("pmc workload done")


def load_traffic():
    """HBM bytes per gemv_kernel launch from the committed counter summary
    (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by the copy calibration)."""
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200, help="timed decode steps (tokens)")
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--configs", default="cfg1,cfg0,cfg2,cfg3,cfg4,export")
    ap.add_argument("--cpu-budget", type=float, default=15.0,
                    help="seconds of reference CPU decode for cpu_baseline (0: skip)")
    ap.add_argument("--pmc-workload", action="store_true",
                    help="run only the workload of the HBM-traffic counter passes")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (see the sharding "
              "notes in the design document); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    import q3vl_int8 as q
    q.lib()  # fails loudly if the HIP library is missing
    torch.cuda.set_device(0)
    if args.pmc_workload:
        pmc_workload()
        return
    configs = args.configs.split(",")
    dims = decode_dims(max_seq=(CTX + args.warmup + args.steps + 7 + 15) // 8 * 8)
    results, cpu, m = [], None, None
    for c in configs:
        log("bench:", c)
        if c == "cfg1":
            m, k16, v16 = build_model(dims, 0xD0C0DE)
            results.append(bench_cfg1(args, m, k16, v16, dims))
        elif c == "cfg0":
            results.append(bench_cfg0(args))
        elif c == "cfg2":
            results.append(bench_cfg2(args))
        elif c == "cfg3":
            results.append(bench_cfg3(args, 1))
            results.append(bench_cfg3(args, 8))
        elif c == "cfg4":
            results.append(bench_cfg4(args))
        elif c == "export":
            results.append(bench_export(args))
        elif c == "load":
            results.append(bench_load(args))
        else:
            raise SystemExit(f"unknown config {c!r} (cfg0..cfg4, export, load)")
        torch.cuda.synchronize()
        log(json.dumps(results[-1]))
    by = {r["name"]: r for r in results}
    head = by.get("cfg1_decode_step")
    if head is None:
        raise SystemExit("the headline needs cfg1 in --configs")
    if args.cpu_budget > 0:
        log("bench: cpu baseline (reference forward_text)")
        cpu = cpu_baseline_cfg1(m, k16, v16, dims, args.cpu_budget)
        if "cfg0_up_proj_gemv" in by:
            by["cfg0_up_proj_gemv"]["cpu_reference"] = cpu_baseline_cfg0(min(5.0, args.cpu_budget))
    rf = head["gemv_roofline"]
    tr = load_traffic()
    line = {
        "metric": "decode tok/s, Qwen3-VL-2B text decoder (int8 group-64 weights), 1 GPU",
        "value": round(head["value"], 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8xi16->i32,f32",
        "data": "synthetic (random-init int8 weights U[-127,127], U(0.001,0.02) group scales; "
                "fp16 KV cache N(0,1) at context 1024)",
        "config": {"workload": "cfg1 greedy decode step: 28 layers, hidden 2048, 16/8 heads x 128, "
                               "intermediate 6144, vocab 151936, group 64, fp16 KV at context 1024, "
                               "batch 1, HIP graph per step",
                   "global_batch": 1, "context": CTX},
        "roofline": {"bound": "hbm", "achieved": round(rf["achieved_GBs"], 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(rf["frac"], 4),
                     "traffic": round(tr["hbm_bytes_per_launch"]) if tr else None,
                     "kernel": rf["kernel"], "bytes_per_launch": round(rf["bytes_per_launch"]),
                     "avg_launch_us": round(rf["avg_launch_us"], 3)},
        "cpu_baseline": cpu,
        "configs": {r["name"]: {k: v for k, v in r.items() if k != "name"} for r in results},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
