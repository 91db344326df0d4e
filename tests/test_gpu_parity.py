"""GPU parity: the HIP library (through its C ABI) against the CPU oracle on the
same seeded inputs. Integer results (q, group sums, argmax ids) and the fp32
outputs of every linear and of SwiGLU (whose expf the device restates from the
host libm's algorithm) are compared bit for bit."""
import ctypes

import numpy as np
import pytest

from golden.gen import make_case, tie_group_row

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
import q3vl_int8 as q  # noqa: E402


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def assert_bits_equal(got, want, what=""):
    g, w = bits(got), bits(want)
    bad = np.flatnonzero(g.ravel() != w.ravel())
    assert bad.size == 0, f"{what}: {bad.size} of {g.size} differ, first at {bad[:5]}: " \
        f"{got.ravel()[bad[:5]]} vs {want.ravel()[bad[:5]]}"


def ulp_diff(a, b):
    ia = bits(a).astype(np.int64)
    ib = bits(b).astype(np.int64)
    ia = np.where(ia >= 2**31, 2**31 - ia, ia)
    ib = np.where(ib >= 2**31, 2**31 - ib, ib)
    return np.abs(ia - ib)


def test_library_is_native():
    assert q.lib()._name == q.LIB_PATH
    assert torch.cuda.is_available()


# ------------------------------------------------------------------ quantizer
@pytest.mark.parametrize("M,K,gs", [(1, 2048, 64), (4, 1024, 16), (3, 2048, 32), (2, 2048, 128),
                                    (2, 4096, 256), (512, 2048, 64), (7, 6144, 64)])
def test_quantize_parity(orc, M, K, gs):
    rng = np.random.default_rng(M * 1000 + gs)
    A = (rng.standard_normal((M, K)) * rng.uniform(0.01, 50, (M, 1))).astype(np.float32)
    A[0, :gs] = 0.0                      # zero group
    if K >= 3 * gs:
        A[0, gs:2 * gs] = 0.3            # constant group
        A[0, 2 * gs:3 * gs] = 0.0
        A[0, 2 * gs + 5] = 7.0           # spike group
    qq, ss = q.quantize_rows(dev(A), gs)
    q_ref, s_ref = orc.quantize_rows(A, gs)
    np.testing.assert_array_equal(host(qq), q_ref)
    assert_bits_equal(host(ss), s_ref, "a_s")


def test_quantize_ties_round_half_even(orc):
    row = tie_group_row(orc)
    qq, ss = q.quantize_rows(dev(row), 64)
    q_ref, s_ref = orc.quantize_rows(row, 64)
    assert s_ref[0, 0] == 1.0
    np.testing.assert_array_equal(host(qq), q_ref)


# --------------------------------------------------------------- linear paths
LANE = [(1, 1024, 1024, 64), (1, 6144, 2048, 64), (1, 2048, 6144, 64), (1, 4096, 2048, 64),
        (1, 1024, 2048, 16), (1, 1024, 2048, 32), (1, 1024, 2048, 128), (1, 1024, 4096, 256),
        (1, 1028, 1024, 64), (1, 1031, 1024, 64), (1, 70000, 1024, 64),
        # K = 2048, group 64 runs blocks of several row tiles: a last tile
        # with one valid row, sub-groups past the last tile, grid strides
        (1, 1029, 2048, 64), (1, 70001, 2048, 64), (1, 2050, 2048, 64)]
GENERAL = [(1, 512, 2048, 64), (1, 2048, 512, 64), (2, 256, 512, 64), (3, 1000, 2048, 64),
           (5, 1028, 1024, 32), (8, 1000, 2048, 64), (8, 384, 6144, 64), (4, 77, 1024, 128),
           (6, 96, 256, 16), (2, 64, 1024, 256),
           # every (rows, threads per group) pair of the reduce-scatter:
           # rows 1, 2, 4, 8 against group sizes 16, 32, 64, 128
           (1, 512, 2048, 128), (1, 256, 1024, 32), (1, 256, 512, 16), (2, 300, 1024, 128),
           (2, 96, 512, 32), (2, 64, 512, 16), (3, 200, 1024, 32), (4, 64, 512, 16),
           (7, 100, 1024, 128)]
GEMM = [(9, 128, 1024, 64), (16, 384, 1024, 64), (64, 512, 2048, 64), (196, 320, 4096, 64),
        (130, 200, 1024, 32), (100, 260, 2048, 128), (512, 2048, 6144, 64)]


def run_linear_case(orc, M, N, K, gs, seed, groups):
    A, W, S = make_case(seed, M, N, K, gs)
    dA, dW, dS = dev(A), dev(W), dev(S)
    G = torch.zeros((M, N, K // gs), dtype=torch.int32, device="cuda") if groups else None
    C = q.linear_i8(dA, dW, dS, gs, groups=G)
    if groups:
        C_ref, G_ref = orc.linear(A, W, S, gs, groups=True)
    else:
        C_ref = orc.linear(A, W, S, gs)
    assert_bits_equal(host(C), C_ref, f"C {M}x{N}x{K} gs{gs}")
    if groups:
        np.testing.assert_array_equal(host(G), G_ref)


@pytest.mark.parametrize("M,N,K,gs", LANE, ids=[str(c) for c in LANE])
def test_lane_gemv_parity(orc, M, N, K, gs):
    assert q.uses_lane_path(M, N, K)
    run_linear_case(orc, M, N, K, gs, seed=N + K + gs, groups=N <= 8192)


# The decode step's row lengths at group 64 without group-sum output: the
# streaming kernel (one wave per row tile, tiles looped per wave), with ragged
# last tiles and more tiles than waves.
# (4100, 5000 and 6144 rows at K = 2048 run 3-row tiles on a 256-CU device,
# the first two with a partial last tile)
STREAM = [(1, 1024, 2048), (1, 1029, 2048), (1, 2050, 2048), (1, 4096, 2048), (1, 9001, 2048),
          (1, 4100, 2048), (1, 5000, 2048), (1, 6144, 2048),
          (1, 1024, 6144), (1, 1031, 6144), (1, 2048, 6144), (1, 6145, 6144)]


@pytest.mark.parametrize("M,N,K", STREAM, ids=[str(c) for c in STREAM])
def test_stream_gemv_parity(orc, M, N, K):
    assert q.uses_lane_path(M, N, K)
    run_linear_case(orc, M, N, K, 64, seed=3 * N + K, groups=False)


@pytest.mark.parametrize("M,N,K,gs", GENERAL, ids=[str(c) for c in GENERAL])
def test_general_gemv_parity(orc, M, N, K, gs):
    assert not q.uses_lane_path(M, N, K)
    run_linear_case(orc, M, N, K, gs, seed=M * 7 + N + K, groups=True)


@pytest.mark.parametrize("M,N,K,gs", GEMM, ids=[str(c) for c in GEMM])
def test_gemm_parity(orc, M, N, K, gs):
    run_linear_case(orc, M, N, K, gs, seed=M + N + K, groups=M * N * K <= 64 * 512 * 2048)


@pytest.mark.parametrize("M,N,K", [(9, 128, 1024), (100, 200, 2048), (130, 260, 1024), (7, 65600, 1024),
                                   (17, 33000, 1024), (64, 512, 512), (300, 700, 1536), (33, 4100, 1536),
                                   (784, 3072, 1024), (196, 2048, 4096), (512, 8192, 1024),
                                   (513, 8200, 1024), (512, 2048, 6144), (1030, 8200, 128),
                                   (1024, 8192, 256), (784, 1024, 1024), (784, 4096, 1024),
                                   (784, 1024, 4096), (196, 4096, 4096)])
def test_gemm_group64_tiles_parity(orc, M, N, K):
    """The group-64 MFMA GEMMs: the fragment-order kernel (K a multiple of
    512) with one m-tile (32 x 128 tiles; 7 rows against the 65600-row
    weight take the 16-row wide kernel) or several (64 x 64 tiles), a
    single w_s tile (K = 512) and an odd number of them (K = 1536), and the
    row-major kernel for the other K; ragged M and N, bit-exact. Every
    vision-encoder linear at its own shape: qkv (784, 3072, 1024), proj
    (784, 1024, 1024), fc1 (784, 4096, 1024), fc2 (784, 1024, 4096), and the
    merger's fc1 (196, 4096, 4096) and fc2 (196, 2048, 4096)."""
    run_linear_case(orc, M, N, K, 64, seed=7 * M + N + K, groups=False)


@pytest.mark.parametrize("M,N,K", [(100, 200, 1024), (333, 1030, 2048), (70, 300, 1536), (1030, 6200, 1024),
                                   (1030, 6200, 128)])
def test_gemm_swiglu_ragged_parity(orc, M, N, K):
    """SwiGLU GEMM: 64 x (64 + 64) tiles with 8-group w_s tiles (SG = 8;
    an odd count, 3, at K = 1536), 128-row tiles once the grid outgrows one
    round of the device (M = 1030), and the row-major kernel at K = 128."""
    A, Wg, Sg = make_case(900 + M, M, N, K, 64)
    _, Wu, Su = make_case(901 + M, M, N, K, 64)
    H = host(q.linear_i8_swiglu(dev(A), dev(Wg), dev(Sg), dev(Wu), dev(Su), 64))
    H_ref = orc.swiglu(orc.linear(A, Wg, Sg, 64), orc.linear(A, Wu, Su, 64))
    np.testing.assert_array_equal(H.view(np.uint32), H_ref.view(np.uint32))


@pytest.mark.parametrize("M,N", [(1, 1030), (3, 700), (40, 300)])
def test_zero_k_gives_zeros(orc, M, N):
    """K = 0: the reference's general path leaves C at zero and the argmax at
    index 0 (the oracle agrees); the library writes them with its zero-fill
    kernel over outputs that held NaN and 77."""
    A = torch.empty((M, 0), dtype=torch.float32, device="cuda")
    W = torch.empty((N, 0), dtype=torch.int8, device="cuda")
    S = torch.empty((N, 0), dtype=torch.float32, device="cuda")
    out = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    C = host(q.linear_i8(A, W, S, 64, out=out))
    C_ref = orc.linear(np.zeros((M, 0), np.float32), np.zeros((N, 0), np.int8),
                       np.zeros((N, 0), np.float32), 64)
    assert_bits_equal(C, C_ref, f"K=0 {M}x{N}")
    ids = torch.full((M,), 77, dtype=torch.int32, device="cuda")
    logits = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    q.lm_head_argmax(A, W, S, 64, logits=logits, ids=ids)
    np.testing.assert_array_equal(host(ids), orc.argmax_rows(C_ref))
    assert_bits_equal(host(logits), C_ref, f"K=0 logits {M}x{N}")


def test_golden_vectors_on_gpu():
    """The reference's own outputs (golden fixtures) reproduced by the GPU."""
    import json
    import os
    from golden.make_golden import LIN_CASES
    gdir = os.path.join(os.path.dirname(__file__), "golden")
    gold = np.load(os.path.join(gdir, "golden_int8.npz"))
    for name, seed, M, N, K, gs in LIN_CASES:
        A, W, S = make_case(seed, M, N, K, gs)
        C = q.linear_i8(dev(A), dev(W), dev(S), gs)
        assert_bits_equal(host(C), gold[f"lin_{name}_C"], name)
    for name, M in (("lane", 1), ("general", 2)):
        A = gold[f"probe_{name}_A"]
        K = A.shape[1]
        C = q.linear_i8(dev(A), dev(np.eye(K, dtype=np.int8)), dev(np.ones((K, K // 64), np.float32)), 64)
        assert_bits_equal(host(C), gold[f"probe_{name}_C"], f"probe {name}")


def test_nonfinite_activation_rows_stay_nonfinite(orc):
    A, W, S = make_case(5, 1, 2048, 2048, 64)
    A[0, 3] = np.nan
    C = host(q.linear_i8(dev(A), dev(W), dev(S), 64))
    C_ref = orc.linear(A, W, S, 64)
    assert np.array_equal(np.isnan(C), np.isnan(C_ref)) and np.isnan(C).all()


@pytest.mark.parametrize("M", [1, 3, 40])
def test_extreme_activation_groups(orc, M):
    """Groups at the edges of the quantizer. Row 0 has only finite group
    scales: squares near fp32 overflow (one element at 1.8e19, q at the
    127 * sqrt(64) bound), 1e18 throughout a group, values at the 1e-6 floor
    of the scale. The GEMV's fast rounding relies on that bound. Row 1 has
    infinite scales (a square that overflows, +-inf) and row 2 a NaN: the
    saturating path (INT32_MIN for NaN products). Bit-exact, NaN where the
    oracle has NaN. M = 40 takes the fragment-order quantizer and the MFMA
    GEMM (its non-finite groups: the saturating branch)."""
    A, W, S = make_case(6, M, 2048, 2048, 64)
    A[0, 0:64] = 1.0e18
    A[0, 5] = -1.7e18
    A[0, 64:128] = 1.0
    A[0, 70] = 1.8e19            # x^2 = 3.24e38 < FLT_MAX
    A[0, 128:192] = 1e-30
    A[0, 192:256] = -3.0
    A[0, 256:320] = 2.5e-3
    A[0, 300] = -7.0e15
    if M > 1:
        A[1, 0:64] = 0.5
        A[1, 10] = 2.0e19        # x^2 overflows: infinite scale
        A[1, 200] = np.inf
        A[1, 330] = -np.inf
        A[2, 384:448] = np.nan
    C = host(q.linear_i8(dev(A), dev(W), dev(S), 64))
    C_ref = orc.linear(A, W, S, 64)
    assert np.isfinite(C_ref[0]).all()
    nan = np.isnan(C_ref)
    assert np.array_equal(np.isnan(C), nan)
    np.testing.assert_array_equal(C[~nan].view(np.uint32), C_ref[~nan].view(np.uint32))


# -------------------------------------------------------------- fused consumers
@pytest.mark.parametrize("M,N,K", [(1, 6144, 2048), (1, 1024, 1024), (4, 512, 1024), (64, 512, 1024),
                                   (512, 768, 2048), (512, 6144, 2048), (300, 8200, 1024),
                                   (1, 1030, 2048), (1, 1027, 2048)])
def test_swiglu_fused_parity(orc, M, N, K):
    gs = 64
    A, Wg, Sg = make_case(100 + M, M, N, K, gs)
    _, Wu, Su = make_case(200 + M, M, N, K, gs)
    H = host(q.linear_i8_swiglu(dev(A), dev(Wg), dev(Sg), dev(Wu), dev(Su), gs))
    g = orc.linear(A, Wg, Sg, gs)
    u = orc.linear(A, Wu, Su, gs)
    H_ref = orc.swiglu(g, u)
    np.testing.assert_array_equal(H.view(np.uint32), H_ref.view(np.uint32))


# The MLP block (q3vl_mlp_i8): fused where M > 8, group 64 and H, I are
# multiples of 512 (the gate|up GEMM's epilogue quantizes h for the down
# GEMM, in its 64-row and, at M = 600 x I = 6144, its 128-row tiles; M = 9
# leaves a block's second m-tile past the product); the two calls through an
# h buffer elsewhere (M <= 8, I = 1088, group 32).
MLP = [(512, 2048, 6144, 64), (100, 1024, 2048, 64), (9, 512, 512, 64), (600, 512, 6144, 64),
       (33, 1024, 1536, 64), (8, 1024, 2048, 64), (64, 1024, 1088, 64), (64, 1024, 1024, 32)]


def mlp_ref(orc, A, Wg, Sg, Wu, Su, Wd, Sd, gs):
    h = orc.swiglu(orc.linear(A, Wg, Sg, gs), orc.linear(A, Wu, Su, gs))
    return orc.linear(h, Wd, Sd, gs)


@pytest.mark.parametrize("M,H,I,gs", MLP, ids=[str(c) for c in MLP])
def test_mlp_parity(orc, M, H, I, gs):
    A, Wg, Sg = make_case(300 + M, M, I, H, gs)
    _, Wu, Su = make_case(301 + M, M, I, H, gs)
    _, Wd, Sd = make_case(302 + M, M, H, I, gs)
    Y = host(q.mlp_i8(dev(A), dev(Wg), dev(Sg), dev(Wu), dev(Su), dev(Wd), dev(Sd), gs))
    assert_bits_equal(Y, mlp_ref(orc, A, Wg, Sg, Wu, Su, Wd, Sd, gs), f"mlp {M}x{H}x{I} gs{gs}")


def test_mlp_extreme_rows(orc):
    """h groups at the quantizer's edges through the fused epilogue: huge
    activations (an h of +-inf or NaN: the saturating branch), tiny ones (the
    1e-6 floor of the scale), with a caller workspace of the advertised size."""
    M, H, I = 40, 512, 512
    A, Wg, Sg = make_case(310, M, I, H, 64)
    _, Wu, Su = make_case(311, M, I, H, 64)
    _, Wd, Sd = make_case(312, M, H, I, 64)
    A[0] = 1.0e18
    A[1] = 1.0e-30
    A[2, :64] = 3.0e5
    A[3, 7] = np.nan
    ws = torch.zeros(q.mlp_workspace_bytes(M, H, I, 64), dtype=torch.uint8, device="cuda")
    Y = host(q.mlp_i8(dev(A), dev(Wg), dev(Sg), dev(Wu), dev(Su), dev(Wd), dev(Sd), 64, workspace=ws))
    Y_ref = mlp_ref(orc, A, Wg, Sg, Wu, Su, Wd, Sd, 64)
    nan = np.isnan(Y_ref)
    assert nan.any() and np.array_equal(np.isnan(Y), nan)
    np.testing.assert_array_equal(Y[~nan].view(np.uint32), Y_ref[~nan].view(np.uint32))


def test_swiglu_standalone(orc):
    from golden.make_golden import swiglu_inputs
    g, u = swiglu_inputs()
    out = host(q.swiglu(dev(g), dev(u)))
    np.testing.assert_array_equal(out.view(np.uint32), orc.swiglu(g, u).view(np.uint32))


def test_swiglu_dense_float_sweep(orc):
    """silu over every 61st fp32 bit pattern (70M gate values, both signs,
    subnormal to infinite) plus inputs whose expf is hardest to round: the
    device expf must equal the host libm's everywhere."""
    bits = np.arange(0, 1 << 32, 61, dtype=np.uint64).astype(np.uint32)
    hard = np.array([-float.fromhex("0x1.04845ep+5"), float.fromhex("0x1.f8cbb2p+5"),
                     -float.fromhex("0x1.fefe02p-16"), 88.7, -88.8, 103.9, 104.0], np.float32)
    g = np.concatenate([bits.view(np.float32), hard])
    u = np.ones_like(g)
    out = host(q.swiglu(dev(g), dev(u)))
    want = orc.swiglu(g, u)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(out), nan)
    np.testing.assert_array_equal(out[~nan].view(np.uint32), want[~nan].view(np.uint32))


@pytest.mark.parametrize("M", [1, 8])
def test_lm_head_argmax_parity(orc, M):
    V, K, gs = 151936, 2048, 64
    A, W, S = make_case(300 + M, M, V, K, gs)
    # plant exact ties: copy the winning row of activation row 0 to a lower
    # and a higher index -> the lowest index must win
    logits_ref = orc.linear(A, W, S, gs)
    top = int(orc.argmax_rows(logits_ref[:1])[0])
    W[top + 7] = W[top]
    S[top + 7] = S[top]
    lo = max(0, top - 1000)
    W[lo] = W[top]
    S[lo] = S[top]
    logits_ref = orc.linear(A, W, S, gs)
    ids_ref = orc.argmax_rows(logits_ref)
    assert ids_ref[0] == lo
    dW, dS, dA = dev(W), dev(S), dev(A)
    logits = torch.empty((M, V), dtype=torch.float32, device="cuda")
    ids = host(q.lm_head_argmax(dA, dW, dS, gs, logits=logits))
    assert_bits_equal(host(logits), logits_ref, "logits")
    np.testing.assert_array_equal(ids, ids_ref)
    ids2 = host(q.lm_head_argmax(dA, dW, dS, gs))  # logits not stored
    np.testing.assert_array_equal(ids2, ids_ref)


@pytest.mark.parametrize("V,off", [(70001, 9), (4099, 5), (151936, 16)])
def test_lm_head_argmax_lane_ties_across_tiles(orc, V, off):
    """M = 1 at K = 2048: the winning row copied `off` rows lower (another
    row tile, worked on by another sub-group of the same block or by another
    block) and 3 rows higher; the lowest index must win. V = 70001 and 4099
    leave a last tile with few valid rows and sub-groups past the end."""
    K, gs = 2048, 64
    A, W, S = make_case(400 + off, 1, V, K, gs)
    top = int(orc.argmax_rows(orc.linear(A, W, S, gs))[0])
    lo = top - off if top >= off else top + 2 * off
    for r in (lo, min(top + 3, V - 1)):
        W[r] = W[top]
        S[r] = S[top]
    logits_ref = orc.linear(A, W, S, gs)
    ids_ref = orc.argmax_rows(logits_ref)
    assert logits_ref[0, lo] == logits_ref[0, top]
    logits = torch.empty((1, V), dtype=torch.float32, device="cuda")
    ids = host(q.lm_head_argmax(dev(A), dev(W), dev(S), gs, logits=logits))
    assert_bits_equal(host(logits), logits_ref, "logits")
    np.testing.assert_array_equal(ids, ids_ref)


@pytest.mark.parametrize("M,V,K", [(12, 5000, 1024), (40, 33000, 2048), (6, 70001, 1024),
                                   (20, 40000, 2048), (32, 33000, 2048)])
def test_lm_head_argmax_gemm_path(orc, M, V, K):
    """lm_head + argmax on the GEMM (then the row argmax): M > 8, and 5..8
    rows against a very wide weight (6 x 70001: the 16-row wide kernel);
    the other single m-tile shapes (M <= 32) take the 1 x 4 wave tiles. A
    planted tie that the lowest index must win, logits bit-exact."""
    gs = 64
    A, W, S = make_case(77 + M, M, V, K, gs)
    top = int(orc.argmax_rows(orc.linear(A[:1], W, S, gs))[0])
    lo = max(0, top - 777)
    W[lo] = W[top]
    S[lo] = S[top]
    logits_ref = orc.linear(A, W, S, gs)
    ids_ref = orc.argmax_rows(logits_ref)
    assert ids_ref[0] == lo
    logits = torch.empty((M, V), dtype=torch.float32, device="cuda")
    ids = host(q.lm_head_argmax(dev(A), dev(W), dev(S), gs, logits=logits))
    assert_bits_equal(host(logits), logits_ref, "logits")
    np.testing.assert_array_equal(ids, ids_ref)


@pytest.mark.parametrize("M,V,K", [(16, 40007, 2048), (13, 65541, 1024), (5, 33000, 2048)])
def test_lm_head_argmax_wide_rows(orc, M, V, K):
    """5..16 rows against a very wide weight (V * K >= 2^26, K <= 2048): the
    16-row MFMA tiles with the weights loaded straight into the operands, one
    argmax partial per wave. V = 40007 and 65541 leave a last tile of 7 and 5
    valid rows. First row 0's winner copied to a column about 2000 lower
    (another wave's tiles) and next to itself: the lowest index must win.
    Then a row of NaN activations (id 0), a column made +-inf/NaN by an
    infinite weight scale and a column of -inf logits for one row. Logits
    bit-exact, ids with and without them stored."""
    gs = 64
    A, W, S = make_case(9100 + M, M, V, K, gs)

    def check(A, W, S):
        logits_ref = orc.linear(A, W, S, gs)
        ids_ref = orc.argmax_rows(logits_ref)
        logits = torch.empty((M, V), dtype=torch.float32, device="cuda")
        ids = host(q.lm_head_argmax(dev(A), dev(W), dev(S), gs, logits=logits))
        np.testing.assert_array_equal(ids, ids_ref)
        got = host(logits)
        nan = np.isnan(logits_ref)
        assert np.array_equal(np.isnan(got), nan)
        np.testing.assert_array_equal(got[~nan].view(np.uint32), logits_ref[~nan].view(np.uint32))
        np.testing.assert_array_equal(host(q.lm_head_argmax(dev(A), dev(W), dev(S), gs)), ids_ref)
        return logits_ref, ids_ref

    top = int(orc.argmax_rows(orc.linear(A[:1], W, S, gs))[0])
    lo = top - 2000 if top >= 2000 else top + 2500
    for r in (lo, min(top + 1, V - 1)):
        W[r] = W[top]
        S[r] = S[top]
    logits_ref, ids_ref = check(A, W, S)
    assert logits_ref[0, lo] == logits_ref[0, top] and ids_ref[0] == min(lo, top)

    A[M - 1, :] = np.nan
    S[17, 3] = np.inf
    W[33, :] = -127
    S[33, :] = np.float32(3e38)
    A[2, :] = np.abs(A[2, :]) + 0.5  # row 2: column 33 -> -inf
    logits_ref, ids_ref = check(A, W, S)
    assert ids_ref[M - 1] == 0 and np.isneginf(logits_ref[2, 33])


@pytest.mark.parametrize("M,N,K", [(9, 36000, 2048), (16, 65539, 1024), (7, 131075, 512)])
def test_linear_wide_rows(orc, M, N, K):
    """The 16-row tiles as a plain product (outputs only, no argmax): every
    K the kernel takes (a tile of 8, 4 and 2 quads of 4 groups), ragged last
    tiles."""
    gs = 64
    A, W, S = make_case(9200 + K, M, N, K, gs)
    assert_bits_equal(host(q.linear_i8(dev(A), dev(W), dev(S), gs)), orc.linear(A, W, S, gs), "C")


def test_lm_head_argmax_partials_over_passes(orc):
    """M = 40 on the GEMM path leaves one argmax partial per 64 columns: at
    V = 140000 that is 2188 partials, more than the final reduction's first
    pass of 2048. Row 0's winner copied into a column of the second pass
    (>= 131072) and to a lower column of the first: the lower one must win
    across the passes; every row's id equals the oracle's scan."""
    M, V, K, gs = 40, 140000, 1024, 64
    A, W, S = make_case(4343, M, V, K, gs)
    top = int(orc.argmax_rows(orc.linear(A[:1], W, S, gs))[0])
    hi, lo = 139000, 5000
    for r in (hi, lo):
        W[r] = W[top]
        S[r] = S[top]
    logits_ref = orc.linear(A, W, S, gs)
    ids_ref = orc.argmax_rows(logits_ref)
    assert ids_ref[0] == min(lo, top) and logits_ref[0, hi] == logits_ref[0, lo]
    ids = host(q.lm_head_argmax(dev(A), dev(W), dev(S), gs))
    np.testing.assert_array_equal(ids, ids_ref)


def test_lm_head_argmax_gemm_special_values(orc):
    """Argmax partials fused into the GEMM: a row of NaN logits (id 0), a
    column made +-inf/NaN by an infinite weight scale, a column whose logits
    are all -inf; ids equal the greedy scan of the oracle's logits, with and
    without the logits stored."""
    M, V, K, gs = 12, 5000, 1024, 64
    A, W, S = make_case(4242, M, V, K, gs)
    A[5, :] = np.nan
    S[17, 3] = np.inf
    W[33, :] = -127
    S[33, :] = np.float32(3e38)
    A[7, :] = np.abs(A[7, :]) + 0.5  # row 7: column 33 -> -inf
    logits_ref = orc.linear(A, W, S, gs)
    ids_ref = orc.argmax_rows(logits_ref)
    assert ids_ref[5] == 0 and np.isneginf(logits_ref[7, 33])
    logits = torch.empty((M, V), dtype=torch.float32, device="cuda")
    ids = host(q.lm_head_argmax(dev(A), dev(W), dev(S), gs, logits=logits))
    np.testing.assert_array_equal(ids, ids_ref)
    got = host(logits)
    nan = np.isnan(logits_ref)
    assert np.array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), logits_ref[~nan].view(np.uint32))
    np.testing.assert_array_equal(host(q.lm_head_argmax(dev(A), dev(W), dev(S), gs)), ids_ref)


def test_argmax_rows_special_values(orc):
    fmax = np.finfo(np.float32).max
    rows = np.full((6, 3000), -np.inf, np.float32)
    rows[1, :] = np.nan
    rows[1, 2000] = 1.0
    rows[2, :] = -fmax
    rows[3, 10] = rows[3, 2999] = 5.0
    rows[4, :] = 0.0
    rows[4, 0] = -0.0
    rows[5] = np.random.default_rng(1).integers(-3, 3, 3000).astype(np.float32)
    ids = host(q.argmax_rows(dev(rows)))
    np.testing.assert_array_equal(ids, orc.argmax_rows(rows))


def test_multi_matches_separate(orc):
    gs, K = 64, 2048
    A, Wq, Sq = make_case(1, 1, 2048, K, gs)
    _, Wk, Sk = make_case(2, 1, 1024, K, gs)
    _, Wv, Sv = make_case(3, 1, 1024, K, gs)
    outs = q.linear_i8_multi(dev(A), [dev(Wq), dev(Wk), dev(Wv)], [dev(Sq), dev(Sk), dev(Sv)], gs)
    for o, (W, S) in zip(outs, [(Wq, Sq), (Wk, Sk), (Wv, Sv)]):
        assert_bits_equal(host(o), orc.linear(A, W, S, gs), "multi")
    # ragged segments (row tiles that straddle no segment end)
    segs = [make_case(5 + i, 1, n, K, gs)[1:] for i, n in enumerate((1030, 1027, 1025))]
    outs = q.linear_i8_multi(dev(A), [dev(W) for W, _ in segs], [dev(S) for _, S in segs], gs)
    for o, (W, S) in zip(outs, segs):
        assert_bits_equal(host(o), orc.linear(A, W, S, gs), "multi ragged")
    # mixed paths (N < 1024 segment with M=1) fall back to separate launches
    _, Ws, Ss = make_case(4, 1, 512, K, gs)
    outs = q.linear_i8_multi(dev(A), [dev(Wq), dev(Ws)], [dev(Sq), dev(Ss)], gs)
    assert_bits_equal(host(outs[1]), orc.linear(A, Ws, Ss, gs), "multi mixed")


def test_caller_workspace(orc):
    M, N, K, gs = 64, 256, 1024, 64
    A, W, S = make_case(8, M, N, K, gs)
    ws = q.alloc_workspace(M, N, K, gs)
    C = q.linear_i8(dev(A), dev(W), dev(S), gs, workspace=ws)
    assert_bits_equal(host(C), orc.linear(A, W, S, gs))
    with pytest.raises(q.Q3VLError) as e:
        q.linear_i8(dev(A), dev(W), dev(S), gs, workspace=ws[:1024])
    assert e.value.code == q.ERR_INVALID_ARGUMENT


def test_error_paths():
    A = torch.zeros((1, 2048 + 4), dtype=torch.float32, device="cuda")
    W = torch.zeros((1024, 2048), dtype=torch.int8, device="cuda")
    S = torch.ones((1024, 32), dtype=torch.float32, device="cuda")
    C = torch.zeros((1, 1024), dtype=torch.float32, device="cuda")
    L = q.lib()
    # misaligned activations (offset by one float)
    rc = L.q3vl_linear_i8(ctypes.c_void_p(A.data_ptr() + 4), ctypes.c_void_p(W.data_ptr()),
                          ctypes.c_void_p(S.data_ptr()), ctypes.c_void_p(C.data_ptr()),
                          1, 1024, 2048, 64, None, 0, None)
    assert rc == q.ERR_INVALID_ARGUMENT and "aligned" in q.last_error()
    # K not a multiple of the group size
    rc = L.q3vl_linear_i8(ctypes.c_void_p(A.data_ptr()), ctypes.c_void_p(W.data_ptr()),
                          ctypes.c_void_p(S.data_ptr()), ctypes.c_void_p(C.data_ptr()),
                          1, 1024, 2000, 64, None, 0, None)
    assert rc == q.ERR_INVALID_ARGUMENT
    # group size the GEMM path does not serve
    rc = L.q3vl_linear_i8(ctypes.c_void_p(A.data_ptr()), ctypes.c_void_p(W.data_ptr()),
                          ctypes.c_void_p(S.data_ptr()), ctypes.c_void_p(C.data_ptr()),
                          16, 8, 1024, 16, None, 0, None)
    assert rc == q.ERR_UNSUPPORTED


def test_dropin_linear_host_pointers(orc):
    """The engine's C++ linear() (host pointers, synchronous) over the GPU."""
    lib = ctypes.CDLL(q.LINEAR_LIB_PATH)
    import subprocess
    sym = [l.split()[-1] for l in subprocess.run(["nm", "-D", q.LINEAR_LIB_PATH], capture_output=True,
                                                  text=True).stdout.splitlines()
           if l.split()[-1].startswith("_Z6linear")][0]
    fn = getattr(lib, sym)
    vp, sz = ctypes.c_void_p, ctypes.c_size_t
    fn.argtypes = [vp, vp, vp, vp, vp, vp, sz, sz, sz, ctypes.c_bool, ctypes.c_int, ctypes.c_int,
                   ctypes.c_int, ctypes.c_int, ctypes.c_bool, sz]
    for (M, N, K) in [(1, 2048, 2048), (3, 512, 1024), (20, 256, 1024)]:
        A, W, S = make_case(N, M, N, K, 64)
        C = np.zeros((M, N), np.float32)
        for _ in range(2):  # second call reuses the registered weight
            fn(A.ctypes.data, W.ctypes.data, S.ctypes.data, None, None, C.ctypes.data, M, N, K, True,
               q.FP32, q.INT8, q.FP32, q.FP32, True, 64)
            assert_bits_equal(C, orc.linear(A, W, S, 64), "drop-in linear")
    q.lib().q3vl_weight_release_all()


def _dropin_linear():
    lib = ctypes.CDLL(q.LINEAR_LIB_PATH)
    import subprocess
    sym = [l.split()[-1] for l in subprocess.run(["nm", "-D", q.LINEAR_LIB_PATH], capture_output=True,
                                                  text=True).stdout.splitlines()
           if l.split()[-1].startswith("_Z6linear")][0]
    fn = getattr(lib, sym)
    vp, sz = ctypes.c_void_p, ctypes.c_size_t
    fn.argtypes = [vp, vp, vp, vp, vp, vp, sz, sz, sz, ctypes.c_bool, ctypes.c_int, ctypes.c_int,
                   ctypes.c_int, ctypes.c_int, ctypes.c_bool, sz]
    return fn


def test_registry_reused_host_address(orc):
    """One host buffer reused for a weight of another shape, then refilled
    with other values: lookup reports the stale entry, the drop-in linear()
    re-uploads and matches the oracle each time."""
    fn = _dropin_linear()
    L = q.lib()
    vp = ctypes.c_void_p
    dW, dS = vp(), vp()
    buf = np.zeros(2048 * 2048, np.int8)       # one host address for every weight
    sbuf = np.zeros(2048 * 2048 // 64, np.float32)
    try:
        for step, (M, N, K, seed) in enumerate([(1, 2048, 2048, 11), (1, 1024, 2048, 12),
                                                (3, 2048, 1024, 13), (3, 2048, 1024, 14)]):
            A, W, S = make_case(seed, M, N, K, 64)
            Wv = buf[:N * K].reshape(N, K)
            Sv = sbuf[:N * K // 64].reshape(N, K // 64)
            Wv[...] = W
            Sv[...] = S
            if step:
                # the previous registration no longer matches this call
                rc = L.q3vl_weight_lookup(Wv.ctypes.data, Sv.ctypes.data, N, K, 64,
                                          ctypes.byref(dW), ctypes.byref(dS))
                assert rc == 5, (step, rc, q.last_error())  # Q3VL_ERR_STALE_WEIGHT
            C = np.zeros((M, N), np.float32)
            fn(A.ctypes.data, Wv.ctypes.data, Sv.ctypes.data, None, None, C.ctypes.data, M, N, K,
               True, q.FP32, q.INT8, q.FP32, q.FP32, True, 64)
            assert_bits_equal(C, orc.linear(A, W, S, 64), f"drop-in linear after reuse {step}")
            assert L.q3vl_weight_lookup(Wv.ctypes.data, Sv.ctypes.data, N, K, 64,
                                        ctypes.byref(dW), ctypes.byref(dS)) == 0
            got = np.empty_like(W)
            hip = ctypes.CDLL("libamdhip64.so")
            hip.hipMemcpy.argtypes = [vp, vp, ctypes.c_size_t, ctypes.c_int]
            assert hip.hipMemcpy(got.ctypes.data, dW, W.nbytes, 2) == 0  # device to host
            assert np.array_equal(got, W), f"registered device copy is stale at step {step}"
        # a wrong scale pointer for a registered weight is stale too
        assert L.q3vl_weight_lookup(buf.ctypes.data, sbuf.ctypes.data + 64, 2048, 1024, 64,
                                    ctypes.byref(dW), ctypes.byref(dS)) == 5
        assert L.q3vl_weight_lookup(buf.ctypes.data + 16, sbuf.ctypes.data, 2048, 1024, 64,
                                    ctypes.byref(dW), ctypes.byref(dS)) == 1
    finally:
        L.q3vl_weight_release_all()
