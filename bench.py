#!/usr/bin/env python3
"""Benchmark of the MI355X int8 group-quantized matmul path.

Prints ONE JSON line (rank 0, N=1). Workloads are BASELINE.json's configs on
synthetic seeded inputs (tests/golden/gen.py distributions), weights resident
in HBM before the timed region:
  cfg0  up_proj GEMV, W int8 [6144, 2048], gs 64             -> GB/s
  cfg2  prefill gate|up (+SwiGLU) [512x2048 -> 2x6144] and down [512x6144 -> 2048]
                                                             -> TOPS (2*M*N*K)
  cfg3  lm_head GEMV + greedy argmax, W [151936, 2048], M=1 and M=8 -> GB/s
The headline (`value`) is the first config in --configs. Each step is one
launch of the hot path over one batch; HBM-bound configs rotate distinct weight
copies so the working set is >2x the 256 MB Infinity Cache. Kernel time is
measured with HIP events on the stream the kernels are launched on.
cpu_baseline: the reference's own linear() (oracle/_ref, compiled from the
reference sources) on the same inputs, timed on this host's cores.
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
INT8_PEAK_TOPS = 5033.0   # dense int8 MFMA (the fp16-MFMA exact path is bound at half)
GS = 64


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _event_time(fn, steps, warmup):
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
    return e0.elapsed_time(e1) / steps  # ms per step


def gen_weights(N, K, copies, seed, device):
    """Random int8 weights uniform in [-127,127] and U(0.001, 0.02) scales,
    generated on the device (seeded)."""
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
    return max(floor, int((600 << 20) // bytes_per_copy) + 1)


def bench_cfg0(args):
    import torch
    import q3vl_int8 as q
    N, K = 6144, 2048
    wbytes = N * K + N * (K // GS) * 4
    n = copies_for(wbytes)
    Ws, Ss = gen_weights(N, K, n, 0xC0FFEE00, "cuda")
    x = torch.randn((1, K), dtype=torch.float32, device="cuda")
    y = torch.empty((1, N), dtype=torch.float32, device="cuda")
    ws = q.alloc_workspace(1, N, K, GS)
    ms = _event_time(lambda i: q.linear_i8(x, Ws[i % n], Ss[i % n], GS, out=y, workspace=ws),
                     args.steps * 20, args.warmup)
    algo = wbytes + K * 4 + N * 4
    gbs = algo / (ms * 1e-3) / 1e9
    return dict(name="cfg0_up_proj_gemv", metric="GB/s", value=gbs, ms=ms, algo_bytes=algo,
                frac=gbs / HBM_PEAK_GBS, copies=n, kernel="gemv_kernel<64,1,true>")


def bench_cfg2(args):
    import torch
    import q3vl_int8 as q
    M, K, I = 512, 2048, 6144
    Wg, Sg = gen_weights(I, K, 1, 1, "cuda")
    Wu, Su = gen_weights(I, K, 1, 2, "cuda")
    Wd, Sd = gen_weights(K, I, 1, 3, "cuda")
    A = torch.randn((M, K), dtype=torch.float32, device="cuda")
    H = torch.empty((M, I), dtype=torch.float32, device="cuda")
    D = torch.empty((M, K), dtype=torch.float32, device="cuda")
    ws = q.alloc_workspace(M, I, max(K, I), GS)

    def step(i):
        q.linear_i8_swiglu(A, Wg[0], Sg[0], Wu[0], Su[0], GS, out=H, workspace=ws)
        q.linear_i8(H, Wd[0], Sd[0], GS, out=D, workspace=ws)

    ms = _event_time(step, args.steps * 5, args.warmup)
    ops = 2 * M * (2 * I) * K + 2 * M * K * I
    tops = ops / (ms * 1e-3) / 1e12
    return dict(name="cfg2_prefill_gemm", metric="TOPS", value=tops, ms=ms, algo_ops=ops,
                frac=tops / INT8_PEAK_TOPS, kernel="quantize + gemm_i8_kernel")


def bench_cfg3(args, M):
    import torch
    import q3vl_int8 as q
    V, K = 151936, 2048
    wbytes = V * K + V * (K // GS) * 4
    n = 3  # 3 x 330 MB > 2x MALL
    Ws, Ss = gen_weights(V, K, n, 0xC0FFEE03, "cuda")
    x = torch.randn((M, K), dtype=torch.float32, device="cuda")
    ids = torch.empty((M,), dtype=torch.int32, device="cuda")
    ws = q.alloc_workspace(M, V, K, GS)
    ms = _event_time(lambda i: q.lm_head_argmax(x, Ws[i % n], Ss[i % n], GS, ids=ids, workspace=ws),
                     args.steps * 4, args.warmup)
    algo = wbytes + M * K * 4 + M * 4
    gbs = algo / (ms * 1e-3) / 1e9
    return dict(name=f"cfg3_lm_head_argmax_m{M}", metric="GB/s", value=gbs, ms=ms, algo_bytes=algo,
                frac=gbs / HBM_PEAK_GBS)


def cpu_baseline_cfg0(budget_s):
    """The reference's linear() (oracle/_ref) on config 0's shape, timed on the
    host cores for about budget_s seconds; falls back to the oracle port."""
    import numpy as np
    from checkers import Oracle, Reference
    from golden.gen import make_case
    N, K = 6144, 2048
    A, W, S = make_case(0xC0FFEE00, 1, N, K, GS)
    ref = Reference.load()
    kind = "reference"
    if ref is None:
        ref, kind = Oracle.load(), "port"
    fn = ref.linear
    fn(A, W, S, GS)
    t0 = time.perf_counter()
    n = 0
    times = []
    while time.perf_counter() - t0 < budget_s:
        t = time.perf_counter()
        fn(A, W, S, GS)
        times.append(time.perf_counter() - t)
        n += 1
    med = float(np.median(times))
    algo = N * K + N * (K // GS) * 4 + K * 4 + N * 4
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)) if kind == "reference" else 1
    return dict(value=algo / med / 1e9, unit="GB/s", cores=threads, kind=kind,
                sample=f"{n} calls of linear() on cfg0 (M=1, N=6144, K=2048, gs=64), median {med*1e3:.3f} ms")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--configs", default="cfg0,cfg2,cfg3")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(the sharding design is described in DESIGN.md); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    import q3vl_int8 as q
    q.lib()
    torch.cuda.set_device(0)
    results = []
    for c in args.configs.split(","):
        log("bench:", c)
        if c == "cfg0":
            results.append(bench_cfg0(args))
        elif c == "cfg2":
            results.append(bench_cfg2(args))
        elif c == "cfg3":
            results.append(bench_cfg3(args, 1))
            results.append(bench_cfg3(args, 8))
        log(json.dumps(results[-1]))
    head = results[0]
    cpu = cpu_baseline_cfg0(args.cpu_budget) if args.cpu_budget > 0 else None
    line = {
        "metric": "int8 GEMV GB/s (cfg0 up_proj, M=1 N=6144 K=2048 gs=64)",
        "value": round(head["value"], 2),
        "unit": head["metric"],
        "n_gpus": 1,
        "steps": args.steps * 20,
        "warmup": args.warmup,
        "ms_per_step": head["ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8xi16->i32,f32",
        "data": "synthetic (seeded int8 U[-127,127] weights, U(0.001,0.02) scales, N(0,1) activations)",
        "config": {"workload": head["name"], "M": 1, "N": 6144, "K": 2048, "group_size": GS},
        "roofline": {"bound": "hbm", "achieved": round(head["value"], 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(head["frac"], 4), "traffic": None},
        "cpu_baseline": cpu,
        "configs": {r["name"]: {k: v for k, v in r.items() if k != "name"} for r in results},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
