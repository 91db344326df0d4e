"""bench.py's CPU leg (no GPU): the reference decode loop stays inside its
caches, the reference step refuses positions past them, and the trace
summary reads a rocprofv3 kernel-trace CSV."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
from golden.gen import SMALL, make_kv_cache, make_text_model  # noqa: E402


def test_cpu_decode_token_cap():
    # the untimed step sits at ctx; timed steps at ctx+1 .. ctx+n < max_seq
    assert bench.cpu_decode_tokens(1024, 1032) == 7
    assert bench.cpu_decode_tokens(1024, 1025) == 0
    assert bench.cpu_decode_tokens(1024, 4096) == bench.CPU_DECODE_TOKENS
    ms = bench.cpu_max_seq(1024)
    assert ms % 8 == 0 and bench.cpu_decode_tokens(1024, ms) == bench.CPU_DECODE_TOKENS


def test_cpu_leg_stops_at_max_seq(ref):
    """max_seq just above the context: the loop runs the 7 steps that fit
    (positions ctx+1 .. max_seq-1) and stops, however long its budget."""
    dims = dict(SMALL, layers=1)
    ctx, max_seq = 40, 48
    r = bench.cpu_leg_cfg1(ref, budget_s=60.0, ctx=ctx, max_seq=max_seq, seed=7, dims=dims)
    assert r["n"] == max_seq - ctx - 1
    assert r["value"] > 0


def test_reference_step_refuses_out_of_range(ref):
    dims = dict(SMALL, layers=1, max_seq=16)
    m = make_text_model(3, dims)
    k16, v16 = make_kv_cache(4, dims, 8)
    dec = ref.decoder(dims, m, k16.astype(np.float32), v16.astype(np.float32))
    try:
        assert np.isfinite(dec.step(5, 15)).all()  # the last row of the cache
        with pytest.raises(ValueError):
            dec.step(5, 16)
        with pytest.raises(ValueError):
            dec.step(dims["vocab"], 9)
        with pytest.raises(ValueError):
            dec.step(-1, 9)
    finally:
        dec.close()


def test_trace_summary(tmp_path):
    """Regions are told apart by their markers' block count (256 threads a
    block): 1 block = the config-1 GEMV region, 3 blocks = config 2."""
    hdr = "Kernel_Name,Grid_Size_X,Grid_Size_Y,Start_Timestamp,End_Timestamp\n"
    rows = [("gemv_kernel<A>", 128, 1, 0, 5000),
            ("swiglu_kernel", 256, 1, 10000, 11000),
            ("gemv_kernel<A>", 128, 1, 12000, 16000),
            ("gemv_kernel<A>", 128, 1, 17000, 23000),
            ("swiglu_kernel", 256, 1, 30000, 31000),
            ("gemv_kernel<A>", 128, 1, 40000, 50000),
            ("swiglu_kernel", 768, 1, 60000, 61000),
            ("gemm_mf_kernel<B>", 4096, 1, 62000, 64000),
            ("swiglu_kernel", 768, 1, 70000, 71000)]
    p = tmp_path / "kt.csv"
    p.write_text(hdr + "".join(f"\"{n}\",{x},{y},{a},{b}\n" for n, x, y, a, b in rows))
    s = bench.trace_summary(str(p))
    assert s["markers"] == 4 and s["dispatches"] == 9
    reg = s["region cfg1_gemv"]["gemv_kernel<A> [128x1]"]
    assert reg["calls"] == 2 and reg["avg_us"] == 5.0
    assert s["region cfg2"]["gemm_mf_kernel<B> [4096x1]"]["calls"] == 1
    assert s["region cfg2 total_us"] == 2.0
    assert s["whole_run"]["gemv_kernel<A> [128x1]"]["calls"] == 4


def test_cpu_info_fields():
    info = bench.cpu_info()
    assert info.get("model")
    assert info.get("physical_cores", 0) >= 1
