// gemm.hip -- int8-weight GEMM for M > 8 on gfx950 matrix cores.
//
// Reference: the general path of linear_int8_fp32s_int32acc_transpose,
// matmul/src/cpu_f32a_i8f32sb_f32c_avx2.cpp:477-662: per output and per
// K-group g (ascending), G = sum_k q[m,k] * w[n,k] exactly in int32, then
//     acc = fma(float(G) * a_s[m,g], w_s[n,g], acc)          (:613-617, 652)
// (GCC contracts the multiply-add; the golden vectors pin this).
//
// Exactness on MFMA. q is int16 with |q| <= 1016, so q and w are exact in
// fp16; every partial sum of one group is an integer below 2^24 in magnitude,
// so v_mfma_f32_32x32x16_f16 accumulating one group in fp32 yields G exactly.
// The accumulator is consumed and cleared at every group boundary by the fp32
// epilogue above, in group order, so C is bit-identical to the reference.
//
// Tiling: block 128(M) x 128(N) x 64(K), 4 waves in 2x2, each wave 64x64 =
// 2x2 MFMA 32x32 tiles. A (fp16) and B (int8) tiles are staged through LDS
// (double buffered, XOR-swizzled 16-byte slots); B is widened to fp16 in
// registers with the 0x64xx exponent trick: half(0x6400|(b^0x80)) - 1152 = b.
// In SwiGLU mode the block's 128 B rows are 64 gate rows and the same 64 up
// rows, and each wave holds a gate tile and the matching up tile so the
// epilogue silu(g)*u needs no exchange.
#include <stdlib.h>

#include "q3vl_device.hpp"
#include "q3vl_kernels.hpp"

namespace q3vl {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int A_STAGE = BM * BK * 2;  // bytes
constexpr int B_STAGE = BN * BK;      // bytes
constexpr int SC_STAGE = 2 * (BM + BN) * 4;  // up to 2 groups of a_s and w_s

// 4 bytes (already xor 0x80) -> 4 fp16 values in two dwords.
__device__ __forceinline__ void widen4(uint32_t x, uint32_t &lo, uint32_t &hi) {
    const uint32_t e = 0x64646464u;
    const uint32_t l = __builtin_amdgcn_perm(e, x, 0x04010400u);
    const uint32_t h = __builtin_amdgcn_perm(e, x, 0x04030402u);
    const half2_t off = {(_Float16)1152.0f, (_Float16)1152.0f};
    lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, l) - off);
    hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, h) - off);
}

template <bool SWIGLU, bool WITH_G>
__global__ __launch_bounds__(256, 2) void gemm_i8_kernel(GemmArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    auto As = [&](int b) { return smem + b * A_STAGE; };
    auto Bs = [&](int b) { return smem + 2 * A_STAGE + b * B_STAGE; };
    auto Sc = [&](int b) {
        return reinterpret_cast<float *>(smem + 2 * A_STAGE + 2 * B_STAGE + b * SC_STAGE);
    };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wid = tid >> 6;
    const int wm = wid & 1, wn = wid >> 1;
    const int l32 = lane & 31, h = lane >> 5;

    const int M = a.M, N = a.N, K = a.K, gs = a.gs;
    const int Kg = K / gs;
    const int m0 = blockIdx.y * BM;
    const int nb = SWIGLU ? BN / 2 : BN;  // output columns per block
    const int n0 = blockIdx.x * nb;
    const int nkb = K / BK;
    const int gpb = gs < BK ? BK / gs : 1;  // groups inside one BK slice

    // ---- staging assignment
    // A: 1024 16-byte chunks (row = c/8, slot = c%8), 4 per thread.
    // B: 512 chunks (row = c/4, slot = c%4), 2 per thread.
    // Row r of the A stage holds activation row m0 + r; chunk c of thread
    // tid + 256 i is (row c/8, 16-byte slot c%8). Offsets are element offsets
    // at k = 0 (32-bit: M*lda and N*K stay below 2^31 by the host checks).
    uint32_t a_off[4];
    int a_dst[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = tid + 256 * i;
        const int row = c >> 3, slot = c & 7;
        const int mrow = min(m0 + row, M - 1);
        a_off[i] = (uint32_t)mrow * (uint32_t)a.lda + slot * 8;
        a_dst[i] = row * 128 + ((slot ^ ((row >> 1) & 7)) << 4);
    }
    // B: row c/4 of the stage, slot c%4. With SWIGLU, stage rows 64..127 are
    // the up rows (thread chunks i=1 cover rows 64..127 exactly).
    uint32_t b_off[2];
    int b_dst[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = tid + 256 * i;
        const int row = c >> 2, slot = c & 3;
        const int nrow = min(n0 + (SWIGLU ? (row & 63) : row), N - 1);
        b_off[i] = (uint32_t)nrow * (uint32_t)K + slot * 16;
        b_dst[i] = row * 64 + ((slot ^ ((row >> 2) & 3)) << 4);
    }
    // scales: thread t < 2*(BM+BN) loads one value per stage
    //   [0, BM*gpb): a_s of group j = t / BM, row t % BM
    //   [2*BM, 2*BM + BN*gpb): w_s of group j, column (t-2BM) % BN
    const int sc_i = tid;  // 256 threads cover 2*(128+128)=512 slots in 2 passes

    u32x4 ra[4], rb[2];
    float rs[2];

    auto load_regs = [&](int kb) {
        const int k0 = kb * BK;
#pragma unroll
        for (int i = 0; i < 4; ++i) ra[i] = *reinterpret_cast<const u32x4 *>(a.Aq + a_off[i] + k0);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int8_t *W = (SWIGLU && i == 1) ? a.W1 : a.W0;
            rb[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(W + b_off[i] + k0));
        }
        const int g0 = k0 / gs;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const int s = sc_i + 256 * p;
            float v = 0.0f;
            if (s < 2 * BM) {
                const int j = s / BM, r = s % BM;
                if (j < gpb) v = a.a_s[(size_t)(g0 + j) * a.lda_s + min(m0 + r, M - 1)];
            } else {
                const int t = s - 2 * BM;
                const int j = t / BN, c = t % BN;
                if (j < gpb) {
                    const float *S;
                    int nrow;
                    if (SWIGLU) {
                        S = c < 64 ? a.S0 : a.S1;
                        nrow = n0 + (c & 63);
                    } else {
                        S = a.S0;
                        nrow = n0 + c;
                    }
                    nrow = min(nrow, N - 1);
                    v = S[(size_t)nrow * Kg + g0 + j];
                }
            }
            rs[p] = v;
        }
    };
    auto store_lds = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4 *>(As(buf) + a_dst[i]) = ra[i];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            u32x4 v = rb[i];
            v ^= (u32x4){0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u};
            *reinterpret_cast<u32x4 *>(Bs(buf) + b_dst[i]) = v;
        }
#pragma unroll
        for (int p = 0; p < 2; ++p) Sc(buf)[sc_i + 256 * p] = rs[p];
    };

    float16_t cacc[2][2], out[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            cacc[i][j] = (float16_t)(0.0f);
            out[i][j] = (float16_t)(0.0f);
        }

    // B row (inside the block tile) of this lane's column for n-tile nt
    int brow[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
        brow[nt] = SWIGLU ? (nt * 64 + wn * 32 + l32) : (wn * 64 + nt * 32 + l32);
    int arow[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) arow[mt] = wm * 64 + mt * 32 + l32;

    load_regs(0);
    store_lds(0);
    __syncthreads();

    for (int kb = 0; kb < nkb; ++kb) {
        const int buf = kb & 1;
        if (kb + 1 < nkb) load_regs(kb + 1);

#pragma unroll
        for (int sp = 0; sp < 2; ++sp) {
            // A fragments: row arow[mt], halves [32sp + 16h, +16) = slots 4sp+2h, +1
            half8_t af[2][2];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                const int r = arow[mt];
                const int sw = (r >> 1) & 7;
                const int s0 = 4 * sp + 2 * h;
                af[mt][0] = *reinterpret_cast<const half8_t *>(As(buf) + r * 128 + ((s0 ^ sw) << 4));
                af[mt][1] =
                    *reinterpret_cast<const half8_t *>(As(buf) + r * 128 + (((s0 + 1) ^ sw) << 4));
            }
            // B fragments: row brow[nt], bytes [32sp + 16h, +16) = slot 2sp+h
            half8_t bf[2][2];
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const int r = brow[nt];
                const int slot = (2 * sp + h) ^ ((r >> 2) & 3);
                const u32x4 raw = *reinterpret_cast<const u32x4 *>(Bs(buf) + r * 64 + (slot << 4));
                uint32_t w[8];
                widen4(raw.x, w[0], w[1]);
                widen4(raw.y, w[2], w[3]);
                widen4(raw.z, w[4], w[5]);
                widen4(raw.w, w[6], w[7]);
                bf[nt][0] = __builtin_bit_cast(half8_t, (u32x4){w[0], w[1], w[2], w[3]});
                bf[nt][1] = __builtin_bit_cast(half8_t, (u32x4){w[4], w[5], w[6], w[7]});
            }
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt)
                        cacc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                            af[mt][u], bf[nt][u], cacc[mt][nt], 0, 0, 0);

            // ---- group boundary: fp32 epilogue in reference order
            const int kend = kb * BK + 32 * sp + 32;  // K consumed so far
            if (kend % gs == 0) {
                const int g = kend / gs - 1;
                const int j = g - (kb * BK) / gs;  // group slot inside this stage
                const float *asT = Sc(buf) + j * BM;
                const float *wsT = Sc(buf) + 2 * BM + j * BN;
#pragma unroll
                for (int mt = 0; mt < 2; ++mt) {
                    float asv[16];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float4 v = *reinterpret_cast<const float4 *>(
                            asT + wm * 64 + mt * 32 + 8 * q + 4 * h);
                        asv[4 * q + 0] = v.x;
                        asv[4 * q + 1] = v.y;
                        asv[4 * q + 2] = v.z;
                        asv[4 * q + 3] = v.w;
                    }
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt) {
                        const float wsv = wsT[brow[nt]];
#pragma unroll
                        for (int e = 0; e < 16; ++e) {
                            const float t = cacc[mt][nt][e] * asv[e];
                            out[mt][nt][e] = fmaf(t, wsv, out[mt][nt][e]);
                        }
                        if (WITH_G) {
                            const int ncol = n0 + brow[nt];
                            if (ncol < N) {
#pragma unroll
                                for (int e = 0; e < 16; ++e) {
                                    const int mrow =
                                        m0 + wm * 64 + mt * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
                                    if (mrow < M)
                                        a.G[((size_t)mrow * N + ncol) * Kg + g] =
                                            (int32_t)cacc[mt][nt][e];
                                }
                            }
                        }
                        cacc[mt][nt] = (float16_t)(0.0f);
                    }
                }
            }
        }

        if (kb + 1 < nkb) store_lds(buf ^ 1);
        __syncthreads();
    }

    // ---- store
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int mrow = m0 + wm * 64 + mt * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
            if (mrow >= M) continue;
            if (SWIGLU) {
                const int ncol = n0 + wn * 32 + l32;
                if (ncol < N)
                    a.C[(size_t)mrow * N + ncol] = silu_mul(out[mt][0][e], out[mt][1][e]);
            } else {
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) {
                    const int ncol = n0 + brow[nt];
                    if (ncol < N) a.C[(size_t)mrow * N + ncol] = out[mt][nt][e];
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// gemm_g64_kernel: the same numerics for group size 64 (the model's), built
// so the matrix cores and the fp32 epilogue overlap.
//
// * One K-step = one group (BK = gs = 64). The group's epilogue is
//   out = fma(float(G)*a_s, w_s, out) in reference order. Two blocks share
//   each CU (240 VGPRs at 128x128), so one wave's VALU epilogue overlaps the
//   other's MFMAs. The first MFMA of a group takes C = 0 (no clearing).
//   (Measured alternatives that did not pay: a second accumulator set per
//   wave to overlap within the wave -- it spills at 128x128 -- and global
//   loads more than one K-step ahead.)
// * B is widened to fp16 once per block when the stage is written to LDS
//   (not once per wave); A arrives as exact fp16 images of the int16
//   activations. Both stages are [rows][64] fp16 with XOR-swizzled 16-byte
//   slots.
// * Scales live in a ring of three LDS slots indexed by group.
// * Tile (32*MT*2) x (32*NT*2), 4 waves in 2x2, each wave (32*MT) x (32*NT);
//   the host picks MT/NT so the grid fills the device. SWIGLU (NT = 2): the
//   block's B rows 0..63 are gate rows, 64..127 the same up rows.
template <int MT, int NT, bool SWIGLU, int D, bool PIPE>
__global__ __launch_bounds__(256, 2) void gemm_g64_kernel(GemmArgs a) {
    constexpr int TBM = 64 * MT, TBN = 64 * NT;
    constexpr int ASTG = TBM * 128, BSTG = TBN * 128;  // bytes per stage (fp16)
    constexpr int SCW = TBM + TBN;                      // floats per scale slot
    constexpr int ACH = TBM * 8 / 256;                  // A 16-byte chunks per thread
    constexpr int BCH = TBN * 4 / 256;                  // B 16-byte int8 chunks per thread
    extern __shared__ __align__(16) unsigned char smem[];
    auto As = [&](int b) { return smem + b * ASTG; };
    auto Bs = [&](int b) { return smem + 2 * ASTG + b * BSTG; };
    float *scr = reinterpret_cast<float *>(smem + 2 * (ASTG + BSTG));  // [3][SCW]

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wm = wid & 1, wn = wid >> 1;
    const int l32 = lane & 31, h = lane >> 5;
    const int M = a.M, N = a.N, K = a.K;
    const int Kg = K / 64;
    const int m0 = blockIdx.y * TBM;
    const int ncols = SWIGLU ? TBN / 2 : TBN;
    const int n0 = blockIdx.x * ncols;

    // ---- staging assignment (element offsets at k = 0)
    uint32_t a_off[ACH];
    int a_dst[ACH];
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
        const int c = tid + 256 * i;
        const int row = c >> 3, slot = c & 7;
        a_off[i] = (uint32_t)min(m0 + row, M - 1) * (uint32_t)a.lda + slot * 8;
        a_dst[i] = row * 128 + ((slot ^ ((row >> 1) & 7)) << 4);
    }
    uint32_t b_off[BCH];
    int b_dst0[BCH], b_dst1[BCH];
    bool b_up[BCH];
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
        const int c = tid + 256 * i;
        const int row = c >> 2, q = c & 3;  // q-th 16 bytes of the row's 64 int8
        const bool up = SWIGLU && row >= 64;
        b_up[i] = up;
        b_off[i] = (uint32_t)min(n0 + (SWIGLU ? (row & 63) : row), N - 1) * (uint32_t)K + q * 16;
        const int s0 = 2 * q, s1 = 2 * q + 1, sw = (row >> 1) & 7;
        b_dst0[i] = row * 128 + ((s0 ^ sw) << 4);
        b_dst1[i] = row * 128 + ((s1 ^ sw) << 4);
    }
    // scale loaders: thread t < TBM loads a_s of row t, TBM <= t < SCW loads
    // w_s of column t - TBM
    // (one unconditional load per thread and K-step: base + kb * stride;
    // threads past SCW read a_s[0] and discard it)
    const bool sc_a = tid < TBM, sc_b = tid >= TBM && tid < SCW;
    const float *sc_base = a.a_s;
    int sc_stride = 0;
    if (sc_a) {
        sc_base = a.a_s + min(m0 + tid, M - 1);
        sc_stride = a.lda_s;
    }
    if (sc_b) {
        const int c = tid - TBM;
        const bool up = SWIGLU && c >= 64;
        sc_base = (up ? a.S1 : a.S0) + (size_t)min(n0 + (SWIGLU ? (c & 63) : c), N - 1) * Kg;
        sc_stride = 1;
    }

    // Global loads run D K-steps ahead through a ring of D register sets
    // (slot = K-step % D; the loop below is unrolled D times so every slot
    // index is a constant). Step kb's slot is free once step kb has been
    // written to LDS, at the end of iteration kb - 1.
    u32x4 ra[D][ACH], rb[D][BCH];
    float rs[D];
    auto load_regs = [&](int slot, int kb) {
        const int k0 = kb * 64;
#pragma unroll
        for (int i = 0; i < ACH; ++i) ra[slot][i] = *reinterpret_cast<const u32x4 *>(a.Aq + a_off[i] + k0);
#pragma unroll
        for (int i = 0; i < BCH; ++i) {
            const int8_t *W = b_up[i] ? a.W1 : a.W0;
            rb[slot][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(W + b_off[i] + k0));
        }
        rs[slot] = sc_base[(size_t)kb * sc_stride];
    };
    auto store_lds = [&](int buf, int slot, int kb) {
#pragma unroll
        for (int i = 0; i < ACH; ++i) *reinterpret_cast<u32x4 *>(As(buf) + a_dst[i]) = ra[slot][i];
#pragma unroll
        for (int i = 0; i < BCH; ++i) {
            u32x4 v = rb[slot][i] ^ (u32x4){0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u};
            uint32_t w[8];
            widen4(v.x, w[0], w[1]);
            widen4(v.y, w[2], w[3]);
            widen4(v.z, w[4], w[5]);
            widen4(v.w, w[6], w[7]);
            *reinterpret_cast<u32x4 *>(Bs(buf) + b_dst0[i]) = (u32x4){w[0], w[1], w[2], w[3]};
            *reinterpret_cast<u32x4 *>(Bs(buf) + b_dst1[i]) = (u32x4){w[4], w[5], w[6], w[7]};
        }
        if (tid < SCW) scr[(kb % 3) * SCW + tid] = rs[slot];
    };

    float16_t acc[MT][NT], out[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) out[mt][nt] = (float16_t)(0.0f);

    int arow[MT], brow[NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) arow[mt] = wm * 32 * MT + mt * 32 + l32;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
        brow[nt] = SWIGLU ? (nt * 64 + wn * 32 + l32) : (wn * 32 * NT + nt * 32 + l32);

    // MFMAs of one K-step (LDS buffer buf) into C
    auto mfma_step = [&](int buf, float16_t (&C)[MT][NT]) {
#pragma unroll
        for (int hs = 0; hs < 2; ++hs) {
            half8_t af[MT][2], bf[NT][2];
            const int s0 = 4 * hs + 2 * h;  // this lane half's 16 k: slots s0, s0+1
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int r = arow[mt], sw = (r >> 1) & 7;
                af[mt][0] = *reinterpret_cast<const half8_t *>(As(buf) + r * 128 + ((s0 ^ sw) << 4));
                af[mt][1] = *reinterpret_cast<const half8_t *>(As(buf) + r * 128 + (((s0 + 1) ^ sw) << 4));
            }
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const int r = brow[nt], sw = (r >> 1) & 7;
                bf[nt][0] = *reinterpret_cast<const half8_t *>(Bs(buf) + r * 128 + ((s0 ^ sw) << 4));
                bf[nt][1] = *reinterpret_cast<const half8_t *>(Bs(buf) + r * 128 + (((s0 + 1) ^ sw) << 4));
            }
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt)
                        C[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                            af[mt][u], bf[nt][u], (hs == 0 && u == 0) ? (float16_t)(0.0f) : C[mt][nt],
                            0, 0, 0);
        }
    };
    // fp32 epilogue of group g from C (reference order)
    auto epilogue = [&](int g, const float16_t (&C)[MT][NT]) {
        const float *asT = scr + (g % 3) * SCW;
        const float *wsT = asT + TBM;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            float asv[16];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 v = *reinterpret_cast<const float4 *>(asT + wm * 32 * MT + mt * 32 + 8 * q + 4 * h);
                asv[4 * q + 0] = v.x;
                asv[4 * q + 1] = v.y;
                asv[4 * q + 2] = v.z;
                asv[4 * q + 3] = v.w;
            }
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const float wsv = wsT[brow[nt]];
#pragma unroll
                for (int e = 0; e < 16; ++e) out[mt][nt][e] = fmaf(C[mt][nt][e] * asv[e], wsv, out[mt][nt][e]);
            }
        }
    };

    const int nkb = K / 64;
    load_regs(0, 0);
    store_lds(0, 0, 0);
#pragma unroll
    for (int j = 1; j < D; ++j) load_regs(j, min(j, nkb - 1));
    __syncthreads();
    if constexpr (PIPE) {
        // Two accumulator sets: step kb's MFMAs (into set kb & 1) are issued
        // before step kb-1's epilogue (from the other set), so the matrix
        // cores and the VALU work at once inside the wave. Epilogues still
        // run in group order; step kb-1's scales stay in their ring slot
        // until step kb+2 is staged.
        float16_t acc2[2][MT][NT];
        constexpr int U = D % 2 == 0 ? D : 2 * D;  // slots and sets both constant
        for (int kb0 = 0; kb0 < nkb; kb0 += U) {
#pragma unroll
            for (int j = 0; j < U; ++j) {
                const int kb = kb0 + j;
                if (kb >= nkb) break;  // uniform
                load_regs(j % D, min(kb + D, nkb - 1));
                mfma_step(kb & 1, acc2[j & 1]);
                if (kb > 0) epilogue(kb - 1, acc2[(j + 1) & 1]);
                if (kb + 1 < nkb) store_lds((kb + 1) & 1, (j + 1) % D, kb + 1);
                __syncthreads();
            }
        }
        // the last step's epilogue (set (nkb - 1) & 1)
        if ((nkb - 1) & 1) epilogue(nkb - 1, acc2[1]);
        else epilogue(nkb - 1, acc2[0]);
    } else {
        for (int kb0 = 0; kb0 < nkb; kb0 += D) {
#pragma unroll
            for (int j = 0; j < D; ++j) {
                const int kb = kb0 + j;
                if (kb >= nkb) break;  // uniform
                // unconditional (the last K-step is reloaded near the end), so
                // the compiler's load counts do not depend on the path taken
                load_regs(j, min(kb + D, nkb - 1));
                mfma_step(kb & 1, acc);
                epilogue(kb, acc);
                if (kb + 1 < nkb) store_lds((kb + 1) & 1, (j + 1) % D, kb + 1);
                __syncthreads();
            }
        }
    }

    // ---- store
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int mrow = m0 + wm * 32 * MT + mt * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
            if (mrow >= M) continue;
            if constexpr (SWIGLU) {
                const int ncol = n0 + wn * 32 + l32;
                if (ncol < N) a.C[(size_t)mrow * N + ncol] = silu_mul(out[mt][0][e], out[mt][1][e]);
            } else {
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    const int ncol = n0 + brow[nt];
                    if (ncol < N) a.C[(size_t)mrow * N + ncol] = out[mt][nt][e];
                }
            }
        }
    }
}

template <int MT, int NT, bool SWIGLU>
static hipError_t launch_g64(const GemmArgs &a, hipStream_t st) {
    // register prefetch depth: as deep as the tile's registers allow
    constexpr int D = MT * NT >= 4 ? 1 : (MT * NT == 2 ? 3 : 4);
    // a second accumulator set (epilogue overlapped with the next MFMAs)
    // where the registers allow it
    constexpr bool PIPE = MT * NT <= 2;
    constexpr int TBM = 64 * MT, TBN = 64 * NT;
    const int ncols = SWIGLU ? TBN / 2 : TBN;
    dim3 grid((a.N + ncols - 1) / ncols, (a.M + TBM - 1) / TBM);
    const size_t lds = 2 * (TBM + TBN) * 128 + 3 * (TBM + TBN) * 4;
    static bool attr_set = false;  // raise the dynamic LDS limit once
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_g64_kernel<MT, NT, SWIGLU, D, PIPE>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    gemm_g64_kernel<MT, NT, SWIGLU, D, PIPE><<<grid, 256, lds, st>>>(a);
    return hipGetLastError();
}

hipError_t launch_gemm(const GemmArgs &a, hipStream_t st) {
    // gs <= 128 keeps every in-group fp32 partial sum below 2^24 (exact).
    if (a.K % BK != 0 || (a.gs != 32 && a.gs != 64 && a.gs != 128))
        return hipErrorInvalidValue;
    if (a.swiglu && a.G) return hipErrorInvalidValue;
    if (a.gs == 64 && !a.G) {
        // tile choice: the largest whose grid covers the device's CUs
        if (a.swiglu) return launch_g64<2, 2, true>(a, st);
        auto tiles = [&](int bm, int bn) { return ((a.M + bm - 1) / bm) * ((a.N + bn - 1) / bn); };
        if (tiles(128, 128) >= 256) return launch_g64<2, 2, false>(a, st);
        if (tiles(64, 128) >= 256) return launch_g64<1, 2, false>(a, st);
        return launch_g64<1, 1, false>(a, st);
    }
    const int nb = a.swiglu ? BN / 2 : BN;
    dim3 grid((a.N + nb - 1) / nb, (a.M + BM - 1) / BM);
    const size_t lds = 2 * (A_STAGE + B_STAGE + SC_STAGE);
    if (a.swiglu) gemm_i8_kernel<true, false><<<grid, 256, lds, st>>>(a);
    else if (a.G) gemm_i8_kernel<false, true><<<grid, 256, lds, st>>>(a);
    else gemm_i8_kernel<false, false><<<grid, 256, lds, st>>>(a);
    return hipGetLastError();
}

}  // namespace q3vl
