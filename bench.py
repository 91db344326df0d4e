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

roofline: the dominant kernels of the decode step, its GEMVs
(gemv_stream_kernel for q|k|v, o, gate|up and down, gemv_kernel for the
lm_head; M=1 lane path), at the decode step's shapes:
achieved = algorithmic bytes (int8 weights + fp32 group scales + fp32
activations in and out) summed over one step's GEMV launches / the summed
kernel durations, measured as HIP-graph replays of each class of launch
between HIP events on the replaying stream; peak = 8 TB/s HBM. In a kernel
trace of this command the roofline region lies between two swiglu_kernel
dispatches (one element each; nothing else in the bench launches that
kernel), so `bench.py --trace-summary <kernel_trace.csv>` gives the same
per-class averages from the profiler's own durations.

cpu_baseline and every config's "cpu_reference": the reference's own code
(oracle/_ref, compiled from the reference sources) on this host's cores,
timed in a child process that runs BEFORE this process touches the GPU (so a
failure there cannot take the GPU figures with it, and no GPU work competes
with it): forward_text on the same random model and context (config 1, fp32
KV cache as the reference keeps it), and linear() at the shapes of configs 0,
2, 3 (M=1 and M=8) and 4, each over a bounded sample stated in its entry.

Also reported under "configs": config 0 (up_proj GEMV, GB/s), config 2
(prefill gate|up+SwiGLU and down at M=512, TOPS), config 3 (lm_head GEMV +
argmax, M=1 and 8, GB/s), config 4 (vision-encoder linears: 24 blocks of
qkv/proj/fc1/fc2 at M=784 and the merger's fc1 and fc2 at M=196, TOPS), the
exporter's weight quantizer on one up_proj ("export", GB/s), the C++
linear() drop-in called with host pointers ("dropin": us per call at config
0's shape, and tok/s over the 197 linears of a decode token) and, with
--configs ...,load, the load of a full-size checkpoint file into HBM (GB/s of
file bytes, page-cache-resident file).
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time
import traceback

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
CPU_DECODE_TOKENS = 200   # cap on the reference decode steps of the CPU leg
MODEL_SEED = 0xD0C0DE
# Vision encoder (config 4): 784 patch tokens, hidden 1024, MLP 4096, 24
# blocks; the 2x2 merger runs over 196 tokens of 4096 (fc1 4096->4096, fc2
# 4096->2048; model/src/load_model.cpp:234-237).
VIS_T, VIS_D, VIS_F, VIS_B = 784, 1024, 4096, 24
VIS_SHAPES = [(3 * VIS_D, VIS_D), (VIS_D, VIS_D), (VIS_F, VIS_D), (VIS_D, VIS_F)]  # (N, K)
MERGER_SHAPES = [(4 * VIS_D, 4 * VIS_D), (2048, 4 * VIS_D)]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def wbytes(N, K):
    return N * K + N * (K // GS) * 4


def cfg2_ops(M=512, K=2048, I=6144):
    return 2 * M * (2 * I) * K + 2 * M * K * I


def vis_block_ops():
    return sum(2 * VIS_T * N * K for N, K in VIS_SHAPES)


def merger_ops():
    return sum(2 * (VIS_T // 4) * N * K for N, K in MERGER_SHAPES)


def cfg4_ops():
    return VIS_B * vis_block_ops() + merger_ops()


# ===================================================================== CPU leg
def cpu_info():
    """CPU model, physical cores and logical CPUs of this host (lscpu, else
    /proc/cpuinfo), and the CPUs this process may run on."""
    info = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        f = {}
        for line in out.splitlines():
            if ":" in line:
                k, v = line.split(":", 1)
                f[k.strip()] = v.strip()
        info["model"] = f.get("Model name")
        if f.get("Core(s) per socket") and f.get("Socket(s)"):
            info["physical_cores"] = int(f["Core(s) per socket"]) * int(f["Socket(s)"])
        if f.get("CPU(s)"):
            info["logical_cpus"] = int(f["CPU(s)"])
    except (OSError, ValueError, subprocess.SubprocessError):
        pass
    if not info.get("model") or not info.get("physical_cores"):
        try:
            cores, model, logical = set(), None, 0
            phys = core = None
            with open("/proc/cpuinfo") as fh:
                for line in fh:
                    k, _, v = line.partition(":")
                    k, v = k.strip(), v.strip()
                    if k == "processor":
                        logical += 1
                    elif k == "model name" and model is None:
                        model = v
                    elif k == "physical id":
                        phys = v
                    elif k == "core id":
                        core = v
                        cores.add((phys, core))
            info.setdefault("model", model)
            if cores:
                info.setdefault("physical_cores", len(cores))
            info.setdefault("logical_cpus", logical)
        except OSError:
            pass
    try:
        info["affinity_cpus"] = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        pass
    info["omp_num_threads"] = os.environ.get("OMP_NUM_THREADS")
    return info


def omp_threads():
    v = os.environ.get("OMP_NUM_THREADS")
    if v and v.isdigit():
        return int(v)
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def _time_calls(fn, budget_s, min_runs=1, max_runs=200):
    """Median wall time of fn() over calls made within budget_s (after one
    untimed call), at least min_runs of them."""
    import numpy as np
    fn()
    times, t0 = [], time.perf_counter()
    while len(times) < max_runs and (len(times) < min_runs or time.perf_counter() - t0 < budget_s):
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    return float(np.median(times)), len(times)


def cpu_decode_tokens(ctx, max_seq, cap=CPU_DECODE_TOKENS):
    """Timed reference decode steps that fit a cache of max_seq positions
    after the untimed step at ctx: positions ctx+1 .. ctx+n must be < max_seq."""
    return max(0, min(cap, max_seq - ctx - 1))


def cpu_max_seq(ctx=CTX, cap=CPU_DECODE_TOKENS):
    """Cache length of the CPU leg's decoder: room for the untimed step at
    ctx and cap timed steps after it."""
    return (ctx + 1 + cap + 7) // 8 * 8


def cpu_leg_cfg1(ref, budget_s, ctx=CTX, max_seq=None, seed=MODEL_SEED, dims=None):
    """forward_text of the reference on the bench's random model at context
    ctx: one untimed step, then greedy steps for about budget_s seconds, never
    past the cache (positions < max_seq)."""
    from golden.gen import QWEN3VL_2B, make_kv_cache, make_text_model
    max_seq = max_seq or cpu_max_seq(ctx)
    dims = dict(dims or QWEN3VL_2B, max_seq=max_seq)
    m = make_text_model(seed, dims)
    k16, v16 = make_kv_cache(seed + 1, dims, ctx)
    k32, v32 = k16.astype("float32"), v16.astype("float32")
    del k16, v16
    dec = ref.decoder(dims, m, k32, v32)
    cap = cpu_decode_tokens(ctx, max_seq)
    try:
        tok = dims["vocab"] - 936
        t0 = time.perf_counter()
        lg = dec.step(tok, ctx)
        first = time.perf_counter() - t0
        n, t0 = 0, time.perf_counter()
        while n < cap and (n == 0 or time.perf_counter() - t0 < budget_s):
            tok = int(lg.argmax())
            lg = dec.step(tok, ctx + 1 + n)
            n += 1
        el = time.perf_counter() - t0
    finally:
        dec.close()
    return dict(value=n / el if n else None, unit="tok/s", n=n, seconds=el,
                sample=f"{n} greedy decode steps of the reference forward_text (28 layers, fp32 KV "
                       f"cache) at contexts {ctx + 1}..{ctx + n}, after one untimed step "
                       f"({first:.2f} s)")


def cpu_leg_linear(ref, budget_s):
    """The reference linear() at the shapes of configs 0, 2, 3 and 4."""
    import numpy as np
    from golden.gen import make_case
    out = {}

    # config 0: up_proj GEMV, M=1 lane path (i8:122-224)
    N, K = 6144, 2048
    A, W, S = make_case(0xC0FFEE00, 1, N, K, GS)
    med, n = _time_calls(lambda: ref.linear(A, W, S, GS), budget_s, min_runs=5)
    algo = wbytes(N, K) + K * 4 + N * 4
    out["cfg0_up_proj_gemv"] = dict(
        value=algo / med / 1e9, unit="GB/s", ms=med * 1e3,
        sample=f"{n} calls of linear() M=1 N=6144 K=2048 (median)")

    # config 2: gate and up (M=512, general path i8:477-662), swiglu, down
    M, H, I = 512, 2048, 6144
    A, Wg, Sg = make_case(0xC0FFEE02, M, I, H, GS)
    _, Wu, Su = make_case(0xC0FFEE12, 1, I, H, GS)
    Ad, Wd, Sd = make_case(0xC0FFEE22, M, H, I, GS)

    def cfg2():
        g = ref.linear(A, Wg, Sg, GS)
        u = ref.linear(A, Wu, Su, GS)
        h = ref.swiglu(g, u)
        ref.linear(h, Wd, Sd, GS)

    med, n = _time_calls(cfg2, budget_s, min_runs=1)
    ops = cfg2_ops(M, H, I)
    out["cfg2_prefill_gemm"] = dict(
        value=ops / med / 1e12, unit="TOPS", ms=med * 1e3,
        sample=f"{n} passes of linear() gate [512x2048 -> 6144], up, swiglu, down [512x6144 -> 2048] "
               f"(median)")

    # config 3: lm_head + greedy argmax, M=1 (huge-N GEMV i8:327-455) and
    # M=8 (general path)
    V = 151936
    _, Wv, Sv = make_case(0xC0FFEE03, 1, V, H, GS)
    for M in (1, 8):
        x = np.random.default_rng(0xC0FFEE13 + M).standard_normal((M, H), dtype=np.float32)

        def cfg3():
            lg = ref.linear(x, Wv, Sv, GS)
            lg.argmax(axis=1)

        med, n = _time_calls(cfg3, budget_s / 2, min_runs=3)
        algo = wbytes(V, H) + M * H * 4 + M * 4
        out[f"cfg3_lm_head_argmax_m{M}"] = dict(
            value=algo / med / 1e9, unit="GB/s", ms=med * 1e3,
            sample=f"{n} calls of linear() M={M} N=151936 K=2048 + argmax of each row (median)")
    del Wv, Sv

    # config 4: a sample of whole ViT blocks (each qkv, proj, fc1, fc2 at
    # M=784 with its own weights) plus the merger's fc1 and fc2 at M=196
    rng = np.random.default_rng(0xC0FFEE04)
    xD = rng.standard_normal((VIS_T, VIS_D), dtype=np.float32)
    xF = rng.standard_normal((VIS_T, VIS_F), dtype=np.float32)
    xM = rng.standard_normal((VIS_T // 4, 4 * VIS_D), dtype=np.float32)
    mw = [make_case(0xC0FFEE40 + j, 1, N, K, GS)[1:] for j, (N, K) in enumerate(MERGER_SHAPES)]
    t_merger = None
    t0 = time.perf_counter()
    for (W, S) in mw:
        ref.linear(xM, W, S, GS)
    t_merger = time.perf_counter() - t0
    blocks, t_blocks = 0, 0.0
    while blocks < VIS_B and (blocks == 0 or t_blocks + t_merger < budget_s):
        ws = [make_case(0xC0FFEE50 + 10 * blocks + j, 1, N, K, GS)[1:]
              for j, (N, K) in enumerate(VIS_SHAPES)]
        t = time.perf_counter()
        for (N, K), (W, S) in zip(VIS_SHAPES, ws):
            ref.linear(xF if K == VIS_F else xD, W, S, GS)
        t_blocks += time.perf_counter() - t
        blocks += 1
    ops = blocks * vis_block_ops() + merger_ops()
    out["cfg4_vision_linears"] = dict(
        value=ops / (t_blocks + t_merger) / 1e12, unit="TOPS", ms=(t_blocks + t_merger) * 1e3,
        sample=f"{blocks} of the 24 ViT blocks (qkv, proj, fc1, fc2 of linear() at M=784) and the "
               f"merger's fc1 and fc2 at M=196, one pass each: {ops / 1e9:.1f} G ops")
    return out


def cpu_leg(args):
    """The child process: every reference CPU figure, as one JSON object."""
    from checkers import Reference
    res = {"cpu": cpu_info(), "threads": omp_threads()}
    ref = Reference.load()
    if ref is None:
        res["error"] = "oracle/_ref/libref_q3vl.so is not built (build() compiles it where the " \
                       "reference sources are present)"
        return res
    budget = args.cpu_budget
    if "cfg1" in args.cpu_configs:
        try:
            res["cfg1_decode_step"] = cpu_leg_cfg1(ref, budget)
        except Exception as e:  # noqa: BLE001 -- reported, the other figures still run
            res["cfg1_decode_step"] = dict(error=repr(e))
    if "linear" in args.cpu_configs:
        try:
            res.update(cpu_leg_linear(ref, max(2.0, budget / 3)))
        except Exception as e:  # noqa: BLE001
            res["linear_error"] = repr(e)
    return res


def run_cpu_leg_child(args):
    """Runs the CPU leg in a child process (this process has not touched the
    GPU yet) and returns its JSON result, or an error record."""
    cmd = [sys.executable, os.path.abspath(__file__), "--cpu-leg", "--cpu-budget",
           str(args.cpu_budget), "--cpu-configs", args.cpu_configs]
    log("bench: cpu leg (reference CPU path, child process):", " ".join(cmd[1:]))
    t = time.perf_counter()
    try:
        p = subprocess.run(cmd, capture_output=True, text=True, timeout=args.cpu_timeout)
    except subprocess.TimeoutExpired:
        return {"error": f"cpu leg exceeded {args.cpu_timeout} s"}
    if p.stderr:
        log(p.stderr.rstrip()[-2000:])
    lines = [ln for ln in p.stdout.splitlines() if ln.startswith("{")]
    if p.returncode != 0 or not lines:
        return {"error": f"cpu leg exited with {p.returncode}", "stdout_tail": p.stdout[-500:]}
    res = json.loads(lines[-1])
    log(f"bench: cpu leg done in {time.perf_counter() - t:.1f} s")
    return res


# =================================================================== GPU legs
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


def _graph_time(fns, reps=5, trials=5, region=None):
    """ms per call of the calls in fns, captured once into a HIP graph and
    replayed (median of `trials` timings of `reps` replays): the kernels'
    own time, without the per-call host overhead of eager launches. With a
    region tag the timed replays sit between that region's trace markers."""
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
    if region:
        region_mark(region)
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
    if region:
        region_mark(region)
    return sorted(out)[len(out) // 2]


# Kernel-trace regions: each timed section is bracketed by two swiglu_kernel
# launches (no bench leg launches that kernel otherwise) of REGION_BLOCKS[tag]
# blocks, so `--trace-summary` attributes the profiler's own durations to the
# section that produced them.
REGION_BLOCKS = {"cfg1_gemv": 1, "cfg0": 2, "cfg2": 3, "cfg3_m1": 4, "cfg3_m8": 5, "cfg4": 6}


def region_mark(tag):
    import torch
    import q3vl_int8 as q
    n = 256 * (REGION_BLOCKS[tag] - 1) + 1
    marker = torch.zeros(n, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    q.swiglu(marker, marker)
    torch.cuda.synchronize()


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


def bench_cfg1(args, m, k16, v16, dims, chunked=False):
    """The decode step in a HIP graph. chunked: the chunked attention order
    (Q3VL_ATTN_CHUNKED) in place of the reference's, reported beside the
    headline (the headline keeps the reference order)."""
    import torch
    from q3vl_int8 import model as qm
    dims = dict(dims, attn_order=qm.ATTN_CHUNKED if chunked else qm.ATTN_REFERENCE)
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
    step_bytes = decode_step_bytes(dims, CTX + args.warmup + args.steps // 2)
    res = dict(name="cfg1_decode_step_chunked_attention" if chunked else "cfg1_decode_step",
               metric="tok/s", value=1000.0 / ms, ms=ms,
               eager_ms=eager_ms, contexts=[CTX + args.warmup, end_pos - 1],
               bytes_per_token=step_bytes, bytes_roofline_tok_s=HBM_PEAK_GBS * 1e9 / step_bytes,
               frac_of_bytes_roofline=(1000.0 / ms) / (HBM_PEAK_GBS * 1e9 / step_bytes),
               kernel_launches_per_token=decode_launches(dims))
    del g
    if chunked:
        res["attention_order"] = ("chunked: per 64-position chunk a max, sum and value chain, folded "
                                  "over the chunks (no counterpart in the reference; within the "
                                  "reference's exp256 error of its order)")
    else:
        res["gemv_roofline"] = decode_gemv_roofline(model, dims)
    return res


def decode_launches(dims):
    """Kernel launches of one q3vl_decode_step: embedding, per layer q|k|v
    GEMV, two attention kernels, o, gate|up and down GEMVs, then the lm_head
    GEMV and the argmax reduction."""
    return 1 + 6 * dims["layers"] + 2


def decode_gemv_shapes(dims):
    """(name, segments [(N, K)]) per GEMV launch of one decode step, as
    q3vl_decode_step issues them."""
    H, I, V = dims["hidden"], dims["inter"], dims["vocab"]
    QD, KD = dims["heads"] * dims["head_dim"], dims["kv_heads"] * dims["head_dim"]
    per_layer = [("qkv", [(QD, H), (KD, H), (KD, H)]), ("o", [(H, QD)]),
                 ("gate_up", [(I, H), (I, H)]), ("down", [(H, I)])]
    return per_layer, ("lm_head", [(V, H)])


def decode_step_bytes(dims, ctx):
    """HBM bytes one decode step must move at context ctx: every weight and
    scale once, the KV cache rows 0..ctx read (fp16) and one row written."""
    per_layer, head = decode_gemv_shapes(dims)
    b = sum(wbytes(N, K) for _, segs in per_layer for N, K in segs) * dims["layers"]
    b += sum(wbytes(N, K) for N, K in head[1])
    kv_row = dims["kv_heads"] * dims["head_dim"] * 2
    return b + dims["layers"] * 2 * kv_row * (ctx + 1)


def decode_gemv_roofline(model, dims):
    """Every GEMV launch of one decode step at its shape, with its layer's
    weights (the lm_head in plain mode). Each class of launch (qkv, o,
    gate/up, down over the 28 layers; lm_head four times) is captured in a
    HIP graph and replayed between HIP events on the capturing stream, so
    time / launches is the average kernel duration (median of five timed
    trials). achieved = one step's algorithmic bytes / one step's summed
    durations. The region is delimited by two one-element swiglu launches,
    its markers in a kernel trace."""
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
    graphs = {}
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
        graphs[name] = g
    region_mark("cfg1_gemv")  # region start (kernel-trace marker)
    st = torch.cuda.current_stream()
    res = {}
    for name, (fns, nbytes) in kinds.items():
        g = graphs[name]
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
        res[name] = dict(us=us, bytes=nbytes, GBs=nbytes / (us * 1e-6) / 1e9,
                         launches_timed=25 * len(fns))
    region_mark("cfg1_gemv")  # region end
    step_us = sum(res[k]["us"] * n for k, n in per_step.items())
    step_bytes = sum(res[k]["bytes"] * n for k, n in per_step.items())
    launches = sum(per_step.values())
    gbs = step_bytes / (step_us * 1e-6) / 1e9
    return dict(kernel="gemv_stream_kernel<KC, MD, R, NW> (q|k|v, o, gate|up, down) and "
                       "gemv_kernel<64, 1, true, 8, 2048, MD, 1> (lm_head): the decode step's GEMV launches",
                launches=launches,
                bytes_per_launch=step_bytes / launches, avg_launch_us=step_us / launches,
                achieved_GBs=gbs, frac=gbs / HBM_PEAK_GBS, step_gemv_us=step_us, by_class=res)


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
    ms = _graph_time([lambda i=i: call(i) for i in range(n)], region="cfg0")
    algo = wbytes(N, K) + K * 4 + N * 4
    gbs = algo / (ms * 1e-3) / 1e9
    return dict(name="cfg0_up_proj_gemv", metric="GB/s", value=gbs, ms=ms, eager_ms=eager_ms,
                algo_bytes=algo, frac=gbs / HBM_PEAK_GBS, copies=n,
                timing="HIP-graph replay of one launch per weight copy (eager_ms: per Python call)",
                kernel="gemv_stream_kernel<2048, 0, 2, 8>")


def bench_dropin(args):
    """The engine's C++ linear() drop-in (matmul/include/hip_wrapper.hpp)
    called as the reference engine calls its CPU linear(): host activations,
    host weights (uploaded once by the weight registry), host output,
    synchronous. q3vl_int8/linear_timing, a native program, times it (a
    Python caller would add its own per-call cost): config 0's shape, and the
    197 linears of one decode token (28 x q, k, v, o, gate, up, down, then
    the lm_head) with every call's host work and waits. Child processes."""
    exe = os.path.join(ROOT, "qwen3-vl-2b-inference_amd", "q3vl_int8", "linear_timing")
    out = dict(name="dropin_linear", metric="us per call / tok/s",
               timing="steady_clock around each linear() call, median; native caller")
    for mode, arg in (("cfg0", "300"), ("seq", "5")):
        r = subprocess.run([exe, mode, arg], capture_output=True, text=True, timeout=300)
        if r.returncode != 0:
            raise RuntimeError(f"linear_timing {mode}: rc {r.returncode}: {r.stderr[-500:]}")
        out[mode] = json.loads(r.stdout.strip().splitlines()[-1])
    out["value"] = out["seq"]["tok_s"]
    return out


def bench_cfg2(args):
    import torch
    import q3vl_int8 as q
    M, K, I = 512, 2048, 6144
    Wg, Sg = gen_weights(I, K, 1, 1)
    Wu, Su = gen_weights(I, K, 1, 2)
    Wd, Sd = gen_weights(K, I, 1, 3)
    A = torch.randn((M, K), dtype=torch.float32, device="cuda")
    D = torch.empty((M, K), dtype=torch.float32, device="cuda")
    ws = torch.zeros(q.mlp_workspace_bytes(M, K, I, GS), dtype=torch.uint8, device="cuda")

    def step():  # the MLP block: gate|up + SwiGLU, then down (q3vl_mlp_i8)
        q.mlp_i8(A, Wg[0], Sg[0], Wu[0], Su[0], Wd[0], Sd[0], GS, out=D, workspace=ws)

    # one HIP graph of the step, replayed: the kernels back to back, without
    # the host time of eager Python calls
    ms = _graph_time([step], reps=10, region="cfg2")
    ops = cfg2_ops(M, K, I)
    tops = ops / (ms * 1e-3) / 1e12
    return dict(name="cfg2_prefill_gemm", metric="TOPS", value=tops, ms=ms, algo_ops=ops,
                frac=tops / FP16_PEAK_TFLOPS, frac_of_int8_peak=tops / INT8_PEAK_TOPS,
                timing="HIP-graph replay of the MLP block (q3vl_mlp_i8: A's quantizer and "
                       "the two GEMMs)",
                kernel="quantize_frag_kernel + gemm_mf_kernel: gate|up with the SwiGLU "
                       "epilogue quantizing h into down's operand, then down")


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
    call = lambda i: q.lm_head_argmax(x, Ws[i % n], Ss[i % n], GS, ids=ids, workspace=ws)
    for i in range(6):  # warm-up
        call(i)
    torch.cuda.synchronize()
    region_mark(f"cfg3_m{M}")
    ms = _event_time(call, max(args.steps // 2, 50), 0)
    region_mark(f"cfg3_m{M}")
    algo = wbytes(V, K) + M * K * 4 + M * 4
    gbs = algo / (ms * 1e-3) / 1e9
    return dict(name=f"cfg3_lm_head_argmax_m{M}", metric="GB/s", value=gbs, ms=ms, algo_bytes=algo,
                frac=gbs / HBM_PEAK_GBS)


def bench_cfg4(args):
    """24 ViT blocks (qkv, proj, fc1, fc2 over 784 patch tokens) and the 2x2
    merger's fc1 and fc2 (196 tokens of 4096): every int8 GEMM of the vision
    encoder with its own random weights."""
    import torch
    import q3vl_int8 as q
    T, D, F, B = VIS_T, VIS_D, VIS_F, VIS_B
    Wb = [[gen_weights(N, K, 1, 7000 + 10 * b + j) for j, (N, K) in enumerate(VIS_SHAPES)]
          for b in range(B)]
    Wm = [gen_weights(N, K, 1, 7990 + j) for j, (N, K) in enumerate(MERGER_SHAPES)]
    xD = torch.randn((T, D), dtype=torch.float32, device="cuda")
    xF = torch.randn((T, F), dtype=torch.float32, device="cuda")
    xM = torch.randn((T // 4, 4 * D), dtype=torch.float32, device="cuda")
    outs = {N: torch.empty((T, N), dtype=torch.float32, device="cuda") for N, _ in VIS_SHAPES}
    outM = {N: torch.empty((T // 4, N), dtype=torch.float32, device="cuda") for N, _ in MERGER_SHAPES}
    ws = q.alloc_workspace(T, 3 * D, F, GS)

    def step():
        for b in range(B):
            for j, (N, K) in enumerate(VIS_SHAPES):
                (W,), (S,) = Wb[b][j]
                q.linear_i8(xF if K == F else xD, W, S, GS, out=outs[N], workspace=ws)
        for j, (N, K) in enumerate(MERGER_SHAPES):
            (W,), (S,) = Wm[j]
            q.linear_i8(xM, W, S, GS, out=outM[N], workspace=ws)

    # one HIP graph of the pass (98 quantizers and 98 GEMMs), replayed
    ms = _graph_time([step], reps=3, region="cfg4")
    ops = cfg4_ops()
    tops = ops / (ms * 1e-3) / 1e12
    return dict(name="cfg4_vision_linears", metric="TOPS", value=tops, ms=ms, algo_ops=ops,
                frac=tops / FP16_PEAK_TFLOPS, frac_of_int8_peak=tops / INT8_PEAK_TOPS,
                gemms=B * len(VIS_SHAPES) + len(MERGER_SHAPES),
                timing="HIP-graph replay of the pass (quantizers and GEMMs)",
                kernel="quantize_frag_kernel + gemm_mf_kernel (K a multiple of 512: every "
                       "vision and merger linear)")


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
    m, k16, v16 = build_model(dims, MODEL_SEED)
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


def pmc_workload_gemm():
    """Workload for the GEMM counter passes: 4 eager calls of each of config
    2's GEMMs (gate|up with the SwiGLU epilogue, then down, M = 512) and of
    config 4's vision linears (qkv, proj, fc1, fc2 at M = 784; the merger's
    fc1 at M = 196), each call its fragment-order quantizer and its
    gemm_mf_kernel."""
    import torch
    import q3vl_int8 as q
    shapes = [("cfg2 gate|up", 512, 6144, 2048, True), ("cfg2 down", 512, 2048, 6144, False)]
    shapes += [(f"cfg4 {n}", VIS_T, N, K, False) for n, (N, K) in zip(("qkv", "proj", "fc1", "fc2"), VIS_SHAPES)]
    shapes += [("cfg4 merger fc1", VIS_T // 4, MERGER_SHAPES[0][0], MERGER_SHAPES[0][1], False)]
    for name, M, N, K, sw in shapes:
        W, S = gen_weights(N, K, 1, 11)
        A = torch.randn((M, K), dtype=torch.float32, device="cuda")
        out = torch.empty((M, N), dtype=torch.float32, device="cuda")
        ws = q.alloc_workspace(M, N, K, GS)
        for _ in range(4):
            if sw:
                W2, S2 = gen_weights(N, K, 1, 12)
                q.linear_i8_swiglu(A, W[0], S[0], W2[0], S2[0], GS, out=out, workspace=ws)
            else:
                q.linear_i8(A, W[0], S[0], GS, out=out, workspace=ws)
        torch.cuda.synchronize()
        log(f"pmc gemm workload: {name} {M}x{N}x{K} done")


def pmc_workload_lmhead():
    """Workload for the lm_head traffic passes: the calibration copy of
    pmc_workload, then 3 calls each of config 3's lm_head + argmax at M = 1
    (gemv_kernel) and M = 8 (gemm_mf_wide_kernel), every call on its own
    weight copy (3 x 331 MB: each streams from HBM)."""
    import torch
    import q3vl_int8 as q
    n = 256 << 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    torch.add(src, 1, out=dst)
    torch.cuda.synchronize()
    del src, dst
    V, K = 151936, 2048
    Ws, Ss = gen_weights(V, K, 3, 0xC0FFEE03)
    for M in (1, 8):
        x = torch.randn((M, K), dtype=torch.float32, device="cuda")
        ids = torch.empty((M,), dtype=torch.int32, device="cuda")
        ws = q.alloc_workspace(M, V, K, GS)
        for i in range(3):
            q.lm_head_argmax(x, Ws[i], Ss[i], GS, ids=ids, workspace=ws)
        torch.cuda.synchronize()
    log("pmc lm_head workload done")


def pmc_kernel_traffic(fetch_dir, write_dir):
    """HBM bytes per dispatch of every kernel in two rocprofv3 --pmc runs of
    a counter workload (FETCH_SIZE, then WRITE_SIZE), each counter scaled by
    what it reads for the workload's calibration copy (256 MiB read, 256 MiB
    written), as pmc_traffic scales the decode GEMVs'."""
    import csv
    import glob

    def per_kernel(d, counter):
        rows = {}
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            with open(f, newline="") as fh:
                for r in csv.DictReader(fh):
                    if r["Counter_Name"] == counter:
                        rows.setdefault(r.get("Kernel_Name", ""), []).append(float(r["Counter_Value"]))
        return rows

    fetch, write = per_kernel(fetch_dir, "FETCH_SIZE"), per_kernel(write_dir, "WRITE_SIZE")
    cands = [(max(v), k) for k, v in fetch.items() if "elementwise" in k]
    if not cands:
        raise SystemExit("no calibration (elementwise) dispatch in the FETCH_SIZE run")
    n_cal = 256 << 20
    ff = n_cal / (max(cands)[0] * 1024)
    wf = n_cal / (max(max(v) for k, v in write.items() if "elementwise" in k) * 1024)
    out = {"calibration": {"fetch_factor": round(ff, 4), "write_factor": round(wf, 4)}}
    for k in sorted(fetch):
        if "elementwise" in k or "distribution" in k:
            continue
        fk = sum(fetch[k]) / len(fetch[k])
        w = write.get(k, [0.0])
        out[k[:120]] = {"dispatches": len(fetch[k]), "fetch_bytes": round(fk * 1024 * ff),
                        "write_bytes": round(sum(w) / len(w) * 1024 * wf)}
    return out


def pmc_summary(dirs, match):
    """Average counter values per dispatch for the kernels whose name holds
    `match`, from rocprofv3 --pmc runs (counter_collection.csv under each
    directory; one run per pass), grouped by kernel name and grid size, with
    the derived figures:
      active_cycles = GRBM_GUI_ACTIVE / 8 (the GRBM count is summed over the
                      8 XCDs: the kernel's own busy cycles on each),
      mfma_busy  = SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs * active_cycles),
      valu_busy  = 4 * SQ_ACTIVE_INST_VALU / (1024 * active_cycles)
                   (SQ_ACTIVE_INST_VALU counts quad-cycles),
      lds_conflict_per_instr = SQ_LDS_BANK_CONFLICT / SQ_INSTS_LDS (stall
                   cycles from LDS bank conflicts per LDS instruction),
      waves_per_simd = SQ_WAVE_CYCLES / SQ_BUSY_CYCLES / 4,
      valu_per_mfma = SQ_INSTS_VALU / SQ_INSTS_MFMA."""
    import csv
    import glob
    vals = {}
    for d in dirs:
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            with open(f, newline="") as fh:
                for r in csv.DictReader(fh):
                    name = r.get("Kernel_Name", "")
                    if match not in name:
                        continue
                    key = f"{name} [grid {r.get('Grid_Size', r.get('Grid_Size_X', '?'))}]"
                    vals.setdefault(key, {}).setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    simds, xcds = 1024, 8
    out = {}
    for key, cs in sorted(vals.items()):
        avg = {c: sum(v) / len(v) for c, v in cs.items()}
        e = dict(dispatches={c: len(v) for c, v in cs.items()}, avg_per_dispatch={c: round(v, 1) for c, v in avg.items()})
        g = avg.get("GRBM_GUI_ACTIVE")
        derived = {}
        if g:
            derived["active_cycles"] = round(g / xcds)
        if g and "SQ_VALU_MFMA_BUSY_CYCLES" in avg:
            derived["mfma_busy"] = round(avg["SQ_VALU_MFMA_BUSY_CYCLES"] / (simds * g / xcds), 4)
        if g and "SQ_ACTIVE_INST_VALU" in avg:
            derived["valu_busy"] = round(4 * avg["SQ_ACTIVE_INST_VALU"] / (simds * g / xcds), 4)
        if avg.get("SQ_INSTS_LDS") and "SQ_LDS_BANK_CONFLICT" in avg:
            derived["lds_conflict_per_instr"] = round(avg["SQ_LDS_BANK_CONFLICT"] / avg["SQ_INSTS_LDS"], 3)
        if avg.get("SQ_BUSY_CYCLES") and "SQ_WAVE_CYCLES" in avg:
            derived["waves_per_simd"] = round(avg["SQ_WAVE_CYCLES"] / avg["SQ_BUSY_CYCLES"] / 4, 3)
        if "SQ_INSTS_VALU" in avg and avg.get("SQ_INSTS_MFMA"):
            derived["valu_per_mfma"] = round(avg["SQ_INSTS_VALU"] / avg["SQ_INSTS_MFMA"], 3)
        e["derived"] = derived
        out[key] = e
    return out


def pmc_traffic(fetch_dir, write_dir):
    """HBM bytes per decode GEMV launch from two rocprofv3 --pmc runs of
    `--pmc-workload` (FETCH_SIZE, then WRITE_SIZE; KiB per dispatch), each
    scaled by what the same counter reads for the workload's calibration copy
    (dst = src + 1 over 256 MiB of uint8: 256 MiB read, 256 MiB written)."""
    import csv
    import glob

    def per_kernel(d, counter):
        rows = {}
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            with open(f, newline="") as fh:
                for r in csv.DictReader(fh):
                    if r["Counter_Name"] == counter:
                        rows.setdefault(r.get("Kernel_Name", ""), []).append(float(r["Counter_Value"]))
        return rows

    fetch, write = per_kernel(fetch_dir, "FETCH_SIZE"), per_kernel(write_dir, "WRITE_SIZE")
    # the calibration copy: the elementwise dispatch that reads the most
    # (torch's fills of the workload's buffers are elementwise too)
    cands = [(max(v), k) for k, v in fetch.items() if "elementwise" in k]
    if not cands:
        raise SystemExit("no calibration (elementwise) dispatch in the FETCH_SIZE run")
    cal = [max(cands)[1]]
    n_cal = 256 << 20
    f_cal = max(fetch[cal[0]])
    w_cal = max(max(v) for k, v in write.items() if "elementwise" in k)
    ff, wf = n_cal / (f_cal * 1024), n_cal / (w_cal * 1024)
    gemv = [k for k in fetch if "gemv" in k]
    nd = sum(len(fetch[k]) for k in gemv)
    fk = sum(sum(fetch[k]) for k in gemv) / nd
    wk = sum(sum(write.get(k, [0.0])) for k in gemv) / nd
    hbm = fk * 1024 * ff + wk * 1024 * wf
    # algorithmic bytes per launch, as decode_gemv_roofline counts them
    # (weights, scales, activations in and out; SwiGLU writes one output)
    dims = decode_dims(max_seq=CTX + 16)
    per_layer, head = decode_gemv_shapes(dims)
    tot = 0
    for name, segs in per_layer:
        K = segs[0][1]
        tot += (sum(wbytes(N, K) for N, _ in segs) + K * 4 +
                (segs[0][0] if name == "gate_up" else sum(N for N, _ in segs)) * 4) * dims["layers"]
    tot += wbytes(*head[1][0]) + head[1][0][1] * 4 + head[1][0][0] * 4
    algo = round(tot / (4 * dims["layers"] + 1))
    return {
        "kernel": "the decode step's GEMVs: q3vl::gemv_stream_kernel<KC, MD, R, NW> (q|k|v, o, "
                  "gate|up, down) and q3vl::gemv_kernel<64, 1, true, 8, 2048, 2, 1> (lm_head)",
        "workload": "3 eager decode steps of config 1 (113 GEMV launches each: q|k|v, o, gate|up, "
                    "down x 28 layers, lm_head)",
        "dispatches": nd,
        "dispatches_by_variant": {k: len(fetch[k]) for k in sorted(gemv)},
        "fetch_size_kib_per_dispatch": round(fk, 1),
        "write_size_kib_per_dispatch": round(wk, 1),
        "calibration": {"kernel": "dst = src + 1 over 256 MiB uint8 (torch elementwise add)",
                        "bytes_read": n_cal, "bytes_written": n_cal,
                        "fetch_size_kib": f_cal, "write_size_kib": w_cal,
                        "fetch_factor": round(ff, 4), "write_factor": round(wf, 4)},
        "hbm_bytes_per_launch": round(hbm),
        "algorithmic_bytes_per_launch": algo,
        "traffic_over_algorithmic": round(hbm / algo, 4),
        "commands": [
            "cd /tmp && TMPDIR=/tmp rocprofv3 --pmc FETCH_SIZE --output-format csv -d "
            "$ROOT/gpurun_out/<fetch_dir> -o run -- python3 $ROOT/bench.py --pmc-workload",
            "cd /tmp && TMPDIR=/tmp rocprofv3 --pmc WRITE_SIZE --output-format csv -d "
            "$ROOT/gpurun_out/<write_dir> -o run -- python3 $ROOT/bench.py --pmc-workload",
            "python3 bench.py --pmc-traffic <fetch_dir> <write_dir>"],
        "other_kernels_same_run": {
            k: {"fetch_kib": round(sum(v) / len(v), 1),
                "write_kib": round(sum(write.get(k, [0.0])) / max(1, len(write.get(k, []))), 1)}
            for k, v in sorted(fetch.items()) if k not in gemv and "elementwise" not in k},
    }


def load_traffic():
    """HBM bytes per gemv_kernel launch from the committed counter summary
    (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by the copy calibration)."""
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


# ============================================================ trace summary
def trace_summary(path):
    """Per-kernel dispatch counts and average durations from a rocprofv3
    kernel trace (CSV), over the whole run and inside the GEMV roofline region
    (between the two swiglu_kernel marker dispatches), grouped by kernel name
    and grid size."""
    import csv
    rows = []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            name = r.get("Kernel_Name") or r.get("KernelName") or ""
            try:
                t0, t1 = int(r["Start_Timestamp"]), int(r["End_Timestamp"])
            except (KeyError, ValueError):
                continue
            grid = "x".join(r.get(k, "?") for k in ("Grid_Size_X", "Grid_Size_Y"))
            rows.append((t0, t1, name, grid))
    rows.sort()
    marks = [i for i, r in enumerate(rows) if "swiglu_kernel" in r[2]]
    tag_of = {v: k for k, v in REGION_BLOCKS.items()}
    regions = {}
    for a, b in zip(marks[0::2], marks[1::2]):
        blocks = rows[a][3].split("x")[0]
        try:
            tag = tag_of.get(int(blocks) // 256, f"grid {blocks}")
        except ValueError:
            tag = f"grid {blocks}"
        regions.setdefault(tag, []).extend(rows[a + 1:b])

    def agg(rs):
        d = {}
        for t0, t1, name, grid in rs:
            e = d.setdefault(f"{name} [{grid}]", [0, 0.0])
            e[0] += 1
            e[1] += (t1 - t0) / 1000.0
        return {k: dict(calls=c, avg_us=round(tot / c, 3), total_us=round(tot, 1))
                for k, (c, tot) in sorted(d.items(), key=lambda kv: -kv[1][1])}

    out = dict(trace=path, dispatches=len(rows), markers=len(marks))
    for tag, rs in regions.items():
        out[f"region {tag}"] = agg(rs)
        out[f"region {tag} total_us"] = round(sum((t1 - t0) / 1000.0 for t0, t1, _, _ in rs), 1)
        # wall time from the region's first dispatch to its last one's end:
        # the timed replays including their launch gaps
        if rs:
            out[f"region {tag} wall_us"] = round((max(t1 for _, t1, _, _ in rs) - rs[0][0]) / 1000.0, 1)
    out["whole_run"] = agg(rows)
    return out


# ===================================================================== main
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200, help="timed decode steps (tokens)")
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--configs", default="cfg1,cfg1c,cfg0,cfg2,cfg3,cfg4,export,dropin")
    ap.add_argument("--cpu-budget", type=float, default=15.0,
                    help="seconds of reference CPU decode for cpu_baseline; the linear() "
                         "figures get a third of it each (0: skip the CPU leg)")
    ap.add_argument("--cpu-configs", default="cfg1,linear",
                    help="CPU figures to time: cfg1 (forward_text), linear (configs 0, 2, 3, 4)")
    ap.add_argument("--cpu-timeout", type=float, default=300.0)
    ap.add_argument("--cpu-leg", action="store_true",
                    help="(internal) run only the reference CPU leg and print its JSON")
    ap.add_argument("--pmc-summary", nargs="+", metavar="DIR",
                    help="print per-dispatch counter averages (and derived GEMM figures) of the "
                         "kernels named by --pmc-match from rocprofv3 --pmc output directories")
    ap.add_argument("--pmc-match", default="gemm_mf_kernel")
    ap.add_argument("--pmc-traffic", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="print the decode GEMVs' HBM traffic summary from the FETCH_SIZE and "
                         "WRITE_SIZE runs of --pmc-workload")
    ap.add_argument("--pmc-workload", nargs="?", const="decode", choices=["decode", "gemm", "lmhead"],
                    help="run only the workload of the counter passes: decode (the decode "
                         "GEMVs' HBM traffic, the default), gemm (configs 2 and 4's GEMMs) or "
                         "lmhead (config 3's lm_head at M = 1 and 8)")
    ap.add_argument("--pmc-kernel-traffic", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="print every kernel's HBM bytes per dispatch from the FETCH_SIZE and "
                         "WRITE_SIZE runs of a --pmc-workload")
    ap.add_argument("--trace-summary", metavar="KERNEL_TRACE_CSV",
                    help="summarize a rocprofv3 kernel trace of this bench and exit")
    args = ap.parse_args()
    if args.trace_summary:
        print(json.dumps(trace_summary(args.trace_summary), indent=1))
        return
    if args.pmc_summary:
        print(json.dumps(pmc_summary(args.pmc_summary, args.pmc_match), indent=1))
        return
    if args.pmc_traffic:
        print(json.dumps(pmc_traffic(*args.pmc_traffic), indent=1))
        return
    if args.pmc_kernel_traffic:
        print(json.dumps(pmc_kernel_traffic(*args.pmc_kernel_traffic), indent=1))
        return
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (see the sharding "
              "notes in the design document); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.cpu_leg:
        print(json.dumps(cpu_leg(args)), flush=True)
        return
    # The CPU leg first, in a child process, before this process touches the GPU.
    cpu_res = run_cpu_leg_child(args) if args.cpu_budget > 0 and not args.pmc_workload else None

    import torch
    import q3vl_int8 as q
    q.lib()  # fails loudly if the HIP library is missing
    torch.cuda.set_device(0)
    if args.pmc_workload:
        {"gemm": pmc_workload_gemm, "lmhead": pmc_workload_lmhead}.get(args.pmc_workload, pmc_workload)()
        return
    configs = args.configs.split(",")
    dims = decode_dims(max_seq=(CTX + args.warmup + args.steps + 7 + 15) // 8 * 8)
    results = []
    runners = {
        "cfg0": lambda: [bench_cfg0(args)],
        "dropin": lambda: [bench_dropin(args)],
        "cfg2": lambda: [bench_cfg2(args)],
        "cfg3": lambda: [bench_cfg3(args, 1), bench_cfg3(args, 8)],
        "cfg4": lambda: [bench_cfg4(args)],
        "export": lambda: [bench_export(args)],
        "load": lambda: [bench_load(args)],
    }
    for c in configs:
        if c not in ("cfg1", "cfg1c") and c not in runners:
            raise SystemExit(f"unknown config {c!r} (cfg0..cfg4, cfg1c, export, load, dropin)")
    decode_model = None
    for c in configs:
        log("bench:", c)
        try:
            if c in ("cfg1", "cfg1c"):
                if decode_model is None:
                    decode_model = build_model(dims, MODEL_SEED)
                m, k16, v16 = decode_model
                out = [bench_cfg1(args, m, k16, v16, dims, chunked=c == "cfg1c")]
                del m, k16, v16
                if not ({"cfg1", "cfg1c"} - set(configs[:configs.index(c) + 1])):
                    decode_model = None  # both decode configs done
            else:
                out = runners[c]()
        except Exception as e:  # noqa: BLE001 -- one config's failure is recorded, not fatal
            traceback.print_exc()
            out = [dict(name=c, error=repr(e))]
        torch.cuda.synchronize()
        for r in out:
            log(json.dumps(r))
        results.extend(out)
        torch.cuda.empty_cache()
    by = {r["name"]: r for r in results}
    head = by.get("cfg1_decode_step") or dict(name="cfg1_decode_step",
                                              error="cfg1 (the headline) not in --configs")

    cpu = None
    if cpu_res is not None:
        threads = cpu_res.get("threads")
        info = cpu_res.get("cpu", {})
        c1 = cpu_res.get("cfg1_decode_step")
        if c1 and c1.get("value"):
            cpu = dict(value=round(c1["value"], 3), unit="tok/s", cores=threads, kind="reference",
                       sample=c1["sample"], cpu_model=info.get("model"),
                       physical_cores=info.get("physical_cores"),
                       logical_cpus=info.get("logical_cpus"))
        else:
            cpu = dict(value=None, unit="tok/s", cores=threads, kind="reference",
                       error=(c1 or {}).get("error") or cpu_res.get("error"))
        for name, r in by.items():
            cr = cpu_res.get(name)
            if cr:
                r["cpu_reference"] = dict(cr, cores=threads, kind="reference",
                                          cpu_model=info.get("model"))
                if cr.get("value") and r.get("value"):
                    r["gpu_over_cpu"] = round(r["value"] / cr["value"], 1)

    rf = head.get("gemv_roofline") if "error" not in head else None
    tr = load_traffic()
    line = {
        "metric": "decode tok/s, Qwen3-VL-2B text decoder (int8 group-64 weights), 1 GPU",
        "value": round(head["value"], 2) if "value" in head else None,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms"], 4) if "ms" in head else None,
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
        "roofline": ({"bound": "hbm", "achieved": round(rf["achieved_GBs"], 1), "peak": HBM_PEAK_GBS,
                      "unit": "GB/s", "frac": round(rf["frac"], 4),
                      "traffic": round(tr["hbm_bytes_per_launch"]) if tr else None,
                      "kernel": rf["kernel"], "bytes_per_launch": round(rf["bytes_per_launch"]),
                      "avg_launch_us": round(rf["avg_launch_us"], 3)} if rf else None),
        "cpu_baseline": cpu,
        "configs": {r["name"]: {k: v for k, v in r.items() if k != "name"} for r in results},
    }
    if "error" in head:
        line["error"] = head["error"]
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
