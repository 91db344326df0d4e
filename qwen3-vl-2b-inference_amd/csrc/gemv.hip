// gemv.hip -- HBM-bound int8 GEMV for M <= 8 (gfx950).
//
// Reference: matmul/src/cpu_f32a_i8f32sb_f32c_avx2.cpp
//   lanes=true  : gemv_lg_N_lg_K_transpose (:122-224) and its huge-N twin
//                 gemv_lg_N_lg_K_transpose_decode (:327-455), taken when
//                 M==1 && N>=1024 && K>=1024 (:464-475);
//   lanes=false : the general path of linear_int8_fp32s_int32acc_transpose
//                 (:477-662) for the remaining M <= 8 shapes.
//
// Work layout. A block has K/16 threads; thread t owns the 16-byte K-chunk t
// of every weight row, so its slice of the quantized activation (8 int16
// pairs per activation row) is computed once and stays in registers while the
// block walks row tiles (R rows, grid-stride). Per row tile every thread issues
// R coalesced 16-byte loads (one per row; a wave reads 1 KiB contiguous).
//   phase 1 (integer): each int8 byte pair is placed in the high bytes of an
//     int16 pair (v_perm) and v_dot2_i32_i16 against the activation pairs
//     gives 256x the exact madd_epi16 lane partials; DPP sums over the gs/16
//     threads of a group give the exact int32 group (lane) sums -> LDS.
//   phase 2 (fp32, reference order): one thread per (row, lane j) [lanes] or
//     per (activation row, weight row) [general] runs the group chain in
//     ascending group order, exactly as the reference's scalar / AVX code.
#include <float.h>
#include <stdlib.h>

#include <mutex>
#include <type_traits>
#include <vector>

#include "q3vl_device.hpp"
#include "q3vl_kernels.hpp"

namespace q3vl {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int GEMV_R = 8;          // weight rows per tile (general path; the lane path picks 2, 4 or 8)
constexpr int GEMV_MAX_THREADS = 512;  // => K <= 8192 on this path
constexpr int GEMV_MAX_GRID = 8192;    // the C ABI reserves this many argmax partials
constexpr int kSubGroups = 4;          // row tiles per block at K = 2048, group 64

// Row stride (in words) of the per-row group buffers: a multiple of 4 whose
// quarter is odd, so 16 lanes reading 16 bytes each at consecutive rows hit
// distinct LDS banks.
__host__ __device__ __forceinline__ int group_ld(int Kg) {
    const int k4 = (Kg + 3) & ~3;
    return ((k4 >> 2) & 1) ? k4 : k4 + 4;
}


// Segment fields held in scalar registers. The kernel never indexes
// a.seg[] with a run-time value: that would fetch the field from kernel
// argument memory with a vector load whose wait also drains every weight
// load in flight.
struct SegRegs {
    const int8_t *W0, *W1, *W2;
    const float *S0, *S1, *S2;
    float *Y0, *Y1, *Y2;
    int32_t *G0, *G1, *G2;
    int N0, N1, N2;
    int t1, t2;  // first tile of segments 1 and 2
};

template <typename T>
__device__ __forceinline__ T pick3(int s, T v0, T v1, T v2) {
    return s == 0 ? v0 : (s == 1 ? v1 : v2);
}

// Rows of one tile: row r is row tn0 + r of segment tseg (plain / argmax), or
// row tn0 + r % (R/2) of the gate (r < R/2) or up segment (swiglu).
struct Tile {
    int tseg, tn0, tN;
};

// Launch kinds with the mode and segment count fixed at compile time.
// (Plain launches keep the run-time form: fixing their segment count
// measured slower for q|k|v and down.)
enum GemvMd : int {
    MD_RUNTIME = 0,
    MD_SWIGLU = 1,   // gate|up with the SwiGLU epilogue
    MD_ARGMAX1 = 2,  // lm_head with the argmax epilogue
};
__host__ __device__ constexpr int md_mode(int md) {
    return md == MD_SWIGLU ? GEMV_SWIGLU : (md == MD_ARGMAX1 ? GEMV_ARGMAX : GEMV_PLAIN);
}
__host__ __device__ constexpr int md_nseg(int md) { return md == MD_SWIGLU ? 2 : 1; }

// The fused norm's chain-major copy of the activation row: 8 rows (one per
// lane chain of the sum of squares), row l holding x[l + 8t] at position t.
// With SEG (row length 2048: 256 positions a chain), each row is cut into 8
// segments of 32 positions with 4 floats of padding after each, so that the
// 64 lanes of a wave, one segment each, read their segments without bank
// conflicts. Words per row:
__host__ __device__ constexpr bool norm_seg(int KC) { return KC == 2048; }
__host__ __device__ constexpr int norm_row_words(int K, bool seg) {
    return seg ? K / 8 + K / 64 + 4 : K / 8 + 4;
}

// KC: the row length K when it is fixed at compile time (the decode step's
// 2048 and 6144), 0 for a run-time K. With KC set, every quantity derived
// from K (group count, LDS layout, index divisions) is a constant.
// MD: the launch's mode and segment count when fixed at compile time
// (GemvMd), so that segment selection folds away; MD_RUNTIME reads them
// from the arguments.
// P: row tiles a block works on side by side. With P > 1 the block is P
// sub-groups of K/16 threads, sub-group p taking tiles blockIdx.x*P + p (grid
// stride gridDim.x*P); the activation row is staged, normalized and quantized
// once for all of them, with the staging spread over the whole block, so a CU
// no longer repeats that work for every resident block. (Decode shapes:
// K = 2048, group 64, one activation row.)
// The segments' weight and scale pointers and first two row counts come
// first, as plain arguments, so that they arrive preloaded in scalar
// registers (kernel-argument preloading takes leading non-aggregate
// arguments only) and the first weight loads wait for no argument fetch.
template <int GS, int MR, bool LANES, int R, int KC, int MD, int P = 1>
__global__ __launch_bounds__(GEMV_MAX_THREADS) void gemv_kernel(
    const int8_t *W0, const int8_t *W1, const int8_t *W2, const float *S0, const float *S1,
    const float *S2, int N0, int N1, GemvArgs a, int ntiles) {
    static_assert(P == 1 || (P == 4 && KC == 2048 && GS == 64 && MR == 1 && LANES),
                  "shared-prologue blocks serve the decode shapes only");
    constexpr int T = GS / 16;
    constexpr int HALF = R / 2;
    // scale values per thread per tile: R*Kg <= (16R/GS) * nthr since nthr >= K/16
    constexpr int SPT = 16 * R >= GS ? 16 * R / GS : 1;
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ float s_norm_inv;

    const int K = KC ? KC : a.K;
    const int Kg = K / GS;
    const int M = a.M;
    // thread index within the sub-group (the K-chunk it owns) and sub-group
    const int tid = P > 1 ? (int)(threadIdx.x & 127) : (int)threadIdx.x;
    // (wave-uniform: a sub-group is two whole waves; readfirstlane keeps the
    // sub-group's tile, segment and row checks in scalar registers)
    const int sub = P > 1 ? __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 7)) : 0;
    const int nthr = KC ? (KC / 16 > 64 ? KC / 16 : 64) : (int)blockDim.x;  // max(K/16, 64)
    const int nchunk = K / 16;
    const bool act = tid < nchunk;   // owns a 16-byte K-chunk
    const int g = act ? tid / T : 0;
    const int tg = tid % T;
    const int mode = MD == MD_RUNTIME ? a.mode : md_mode(MD);
    const bool swg = mode == GEMV_SWIGLU;

    SegRegs sr;
    sr.W0 = W0; sr.W1 = W1; sr.W2 = W2;
    sr.S0 = S0; sr.S1 = S1; sr.S2 = S2;
    sr.Y0 = a.seg[0].Y; sr.Y1 = a.seg[1].Y; sr.Y2 = a.seg[2].Y;
    sr.G0 = a.seg[0].G; sr.G1 = a.seg[1].G; sr.G2 = a.seg[2].G;
    sr.N0 = N0; sr.N1 = N1; sr.N2 = a.seg[2].N;
    const float *Ap = a.A;
    const int8_t *norm_w = a.norm_w;
    const float *norm_s = a.norm_s;
    int nseg = MD == MD_RUNTIME ? a.nseg : md_nseg(MD);
    // The integer kernel arguments are read here, in the entry batch of
    // scalar loads: the opaque copies keep the compiler from re-loading them
    // later (its cost model treats a kernel-argument load as free to repeat),
    // each re-load a dependent round trip. (Pointers are left alone: an
    // opaque copy would lose their global address space.)
    asm volatile("" : "+s"(sr.N0), "+s"(sr.N1), "+s"(sr.N2));
    if constexpr (MD == MD_RUNTIME) asm volatile("" : "+s"(nseg));
    sr.t1 = (sr.N0 + R - 1) / R;
    sr.t2 = nseg > 2 ? sr.t1 + (sr.N1 + R - 1) / R : 0x7fffffff;
    if (nseg < 2) sr.t1 = 0x7fffffff;

    auto resolve = [&](int tile) {
        Tile t;
        if (swg) {
            t.tseg = 0;
            t.tn0 = tile * HALF;
            t.tN = sr.N0;
        } else {
            t.tseg = tile < sr.t1 ? 0 : (tile < sr.t2 ? 1 : 2);
            t.tn0 = (tile - pick3(t.tseg, 0, sr.t1, sr.t2)) * R;
            t.tN = pick3(t.tseg, sr.N0, sr.N1, sr.N2);
        }
        return t;
    };
    auto row_seg = [&](const Tile &t, int r) { return swg ? (r < HALF ? 0 : 1) : t.tseg; };
    auto row_n = [&](const Tile &t, int r) { return swg ? t.tn0 + (r & (HALF - 1)) : t.tn0 + r; };
    auto row_ok = [&](const Tile &t, int r) { return row_n(t, r) < t.tN; };
    auto seg_W = [&](int s) { return pick3(s, sr.W0, sr.W1, sr.W2); };
    auto seg_S = [&](int s) { return pick3(s, sr.S0, sr.S1, sr.S2); };
    auto seg_Y = [&](int s) { return pick3(s, sr.Y0, sr.Y1, sr.Y2); };
    auto seg_G = [&](int s) { return pick3(s, sr.G0, sr.G1, sr.G2); };

    // ---- LDS carve-up. accb holds the exact integer sums, one padded row of
    // ld words per chain: [r*8 + lane][g] (lanes) or [m*R + r][g] (general).
    const int ld = group_ld(Kg);
    const int acc_words = (LANES ? 8 * R : MR * R) * ld;
    // >= K (activation staging, 4 float4 per thread: 16*nthr words), plus
    // the chain-major copy of the row for a fused norm (8 rows of K/8 + 4),
    // and >= 2*nthr (argmax scratch)
    const bool has_norm = norm_w != nullptr;
    constexpr bool SEGN = norm_seg(KC);
    const int nrs = norm_row_words(K, SEGN);
    // The staged row keeps 4 floats of padding after every group, so the
    // threads of a wave, each reading its own group, hit distinct banks.
    const int xpad = 4 * (16 * nthr / GS);
    const int stage_need = 16 * nthr + xpad + (has_norm ? 8 * nrs : 0);
    // (one accb per sub-group; all of them alias the phase-0 staging)
    const int stage_words = P * acc_words > stage_need ? P * acc_words : stage_need;
    int32_t *accb = reinterpret_cast<int32_t *>(smem) + sub * acc_words;
    float *xs = reinterpret_cast<float *>(smem);  // phase 0 only (aliases accb)
    float *xn = xs + 16 * nthr + xpad;            // [8][nrs]: x[l + 8j] at l*nrs + j
    // element e of the staged row (groups padded by 4 floats)
    auto xpos = [&](int e) { return e + 4 * (e / GS); };
    float *as_l = reinterpret_cast<float *>(smem) + stage_words;  // [M][Kg]
    // P > 1: the quantized row, 8 words (16 int16) per K-chunk, handed from
    // the threads that quantize it to every sub-group
    uint32_t *qs = reinterpret_cast<uint32_t *>(as_l + MR * Kg);
    float *sc_l = reinterpret_cast<float *>(qs + (P > 1 ? 8 * nthr : 0)) + sub * R * ld;  // [P][R][ld]
    float *ybuf = reinterpret_cast<float *>(qs + (P > 1 ? 8 * nthr : 0)) + P * R * ld + sub * MR * R;  // [P][MR][R]

    // Weight chunk and scale prefetch for one tile (registers).
    u32x4 wv[R];
    float sv[SPT];
    // Rows past the segment end and idle threads read a safe address (row 0,
    // chunk 0) whose value is never used: no select on loaded data, so no
    // wait is forced at issue time.
    // Scales first, then weights: the scale fill at the top of the next
    // iteration then waits only for the scales (vmcnt retires in order).
    auto prefetch = [&](const Tile &t) {
#pragma unroll
        for (int j = 0; j < SPT; ++j) {
            const int i = tid + j * nthr;
            const int r = i / Kg, gg = i - (i / Kg) * Kg;
            const bool ok = i < R * Kg && row_ok(t, r);
            const int sg = swg ? (r < HALF ? 0 : 1) : t.tseg;
            sv[j] = seg_S(sg)[ok ? (size_t)row_n(t, r) * Kg + gg : 0];
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const bool ok = act && row_ok(t, r);
            const int8_t *w = seg_W(row_seg(t, r)) + (size_t)(ok ? row_n(t, r) : 0) * K + 16 * (ok ? tid : 0);
            wv[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(w));
        }
    };

    // this sub-group's first tile; a block's sub-groups advance together (a
    // sub-group past the last tile runs it with no valid rows), so every
    // barrier below is reached by the whole block
    int tile = blockIdx.x * P + sub;

    // ---- phase 0: quantize the activation rows (reference i8:135-177).
    // Row 0's loads are issued before the first tile's weight loads so that
    // waiting for them does not wait for the weights.
    //
    // The fused norm's chain-major copy of float4 i of the staged row:
    // element 4i + c sits in chain 4*(i&1) + c at i/2.
    auto put4 = [&](int i, const float4 &v) {
        if (i < K / 4) {
            const int t = i >> 1;  // position in the chain
            float *d = xn + 4 * (i & 1) * nrs + (SEGN ? t + 4 * (t >> 5) : t);
            d[0] = v.x;
            d[nrs] = v.y;
            d[2 * nrs] = v.z;
            d[3 * nrs] = v.w;
        }
    };
    // The fused norm: sum of squares in the reference's 8-lane order (lanes
    // 0..7 of the block's wave 0), then inv = 1/sqrt(ss/K + eps) in fp32.
    auto norm_chain = [&]() {
        if (SEGN && threadIdx.x < 64) {
            // lane 8l + j holds segment j (positions 32j .. 32j+31) of
            // chain l in registers. Segment s: every lane runs its 32
            // FMAs, but only lanes j == s carry their chain (the others'
            // sums are discarded); a row shift then hands each chain's
            // sum to the lane of its next segment. So chain l is the
            // reference's FMA sequence over t = 0..255, with no LDS read
            // between its FMAs.
            const float *sg = xn + (tid >> 3) * nrs + (tid & 7) * 36;
            float4 X[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) X[u] = reinterpret_cast<const float4 *>(sg)[u];
            float acc = 0.0f;
#pragma unroll
            for (int sgm = 0; sgm < 8; ++sgm) {
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    acc = fmaf(X[u].x, X[u].x, acc);
                    acc = fmaf(X[u].y, X[u].y, acc);
                    acc = fmaf(X[u].z, X[u].z, acc);
                    acc = fmaf(X[u].w, X[u].w, acc);
                }
                if (sgm < 7)  // row_shr:1 (lane i takes lane i-1 inside each row of 16)
                    acc = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                              0, __builtin_bit_cast(int, acc), 0x111, 0xF, 0xF, false));
            }
            // chain l's sum sits in lane 8l + 7; added in chain order
            float ss = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), 7));
#pragma unroll
            for (int l = 1; l < 8; ++l)
                ss = ss + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), 8 * l + 7));
            if (threadIdx.x == 0) s_norm_inv = rcp_rn(sqrt_rn(ss * rcp_rn((float)K) + a.norm_eps));
        } else if (threadIdx.x < 64) {
            float acc = 0.0f;
            if (tid < 8) {
                const float *row = xn + tid * nrs;
                const int cnt = K / 8;
                // batches of 32 in two register sets used in turn: the
                // next batch's reads are in flight during this batch's
                // FMAs (s_waitcnt lgkmcnt(0) before issuing them: two
                // batches of 8 reads exceed what the 4-bit counter tells
                // apart)
                float4 A[8], B[8];
                auto ld = [&](float4 *D, int i) {
#pragma unroll
                    for (int u = 0; u < 8; ++u) D[u] = reinterpret_cast<const float4 *>(row + i)[u];
                };
                auto sq = [&](const float4 *D) {
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        acc = fmaf(D[u].x, D[u].x, acc);
                        acc = fmaf(D[u].y, D[u].y, acc);
                        acc = fmaf(D[u].z, D[u].z, acc);
                        acc = fmaf(D[u].w, D[u].w, acc);
                    }
                };
                int j = 0;
                if (cnt >= 32) {
                    ld(A, 0);
                    for (; j + 64 <= cnt; j += 64) {
                        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
                        __builtin_amdgcn_sched_barrier(0);
                        ld(B, j + 32);
                        sq(A);
                        __builtin_amdgcn_sched_barrier(0);
                        __builtin_amdgcn_s_waitcnt(0xC07F);
                        __builtin_amdgcn_sched_barrier(0);
                        ld(A, j + 64 + 32 <= cnt ? j + 64 : j);  // (re-read when no batch is left)
                        sq(B);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                    if (j + 32 <= cnt) {  // A holds j .. j+31
                        __builtin_amdgcn_s_waitcnt(0xC07F);
                        sq(A);
                        j += 32;
                    }
                }
                for (; j < cnt; ++j) acc = fmaf(row[j], row[j], acc);
            }
            float ss = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), 0));
#pragma unroll
            for (int l = 1; l < 8; ++l)
                ss = ss + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), l));
            if (threadIdx.x == 0) s_norm_inv = rcp_rn(sqrt_rn(ss * rcp_rn((float)K) + a.norm_eps));
        }
    };
    uint32_t qp[MR][8];
    // The quantizer of K-chunk tid of activation row m.
    auto quant_chunk = [&](int m) {
        // The group's sum of squares in the reference order: 16 FMA
        // chains (chain c takes elements 16t + c over the gs/16 steps t),
        // V[i] = P[i] + P[i+8], then the fixed tree.
        float sumsq;
        if constexpr (T == 4) {
            // The group's 4 threads are one lane quad; thread tg runs
            // chains 4tg .. 4tg+3 (one 16-byte read per step). Lanes 0/1
            // take the P[i+8] of lanes 2/3, and lane 0 takes lane 1's
            // half of V (DPP quad permutes): the same adds in the same
            // order, with 4 LDS reads instead of the whole group.
            const float *xg = xs + g * (GS + 4);
            float4 cv[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) cv[t] = *reinterpret_cast<const float4 *>(xg + 16 * t + 4 * tg);
            float p0 = 0.0f, p1 = 0.0f, p2 = 0.0f, p3 = 0.0f;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                p0 = fmaf(cv[t].x, cv[t].x, p0);
                p1 = fmaf(cv[t].y, cv[t].y, p1);
                p2 = fmaf(cv[t].z, cv[t].z, p2);
                p3 = fmaf(cv[t].w, cv[t].w, p3);
            }
#define Q3VL_QUAD(v, ctrl) \
__builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), ctrl, 0xF, 0xF, false))
            // quad_perm [2,3,2,3]: lanes 0, 1 read lanes 2, 3
            const float v0 = p0 + Q3VL_QUAD(p0, 0xEE), v1 = p1 + Q3VL_QUAD(p1, 0xEE);
            const float v2 = p2 + Q3VL_QUAD(p2, 0xEE), v3 = p3 + Q3VL_QUAD(p3, 0xEE);
            // quad_perm [1,1,1,1]: lane 1's V[4..7]
            const float w0 = Q3VL_QUAD(v0, 0x55), w1 = Q3VL_QUAD(v1, 0x55);
            const float w2 = Q3VL_QUAD(v2, 0x55), w3 = Q3VL_QUAD(v3, 0x55);
            // lane 0's value to the quad (quad_perm [0,0,0,0])
            sumsq = Q3VL_QUAD(tree8(v0, v1, v2, v3, w0, w1, w2, w3), 0x00);
#undef Q3VL_QUAD
        } else {
            // every thread of the group runs all 16 chains from LDS (all
            // of the group's reads are issued before the first FMA: one
            // read latency instead of one per pair of reads)
            float Pc[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) Pc[i] = 0.0f;
            const float *xg = xs + g * (GS + 4);
            constexpr int TB = T < 4 ? T : 4;  // sub-blocks of 16 read per batch
#pragma unroll
            for (int t0 = 0; t0 < T; t0 += TB) {
                float4 vb[TB][4];
#pragma unroll
                for (int t = 0; t < TB; ++t)
#pragma unroll
                    for (int i4 = 0; i4 < 4; ++i4)
                        vb[t][i4] = reinterpret_cast<const float4 *>(xg + 16 * (t0 + t))[i4];
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int t = 0; t < TB; ++t) {
#pragma unroll
                    for (int i4 = 0; i4 < 4; ++i4) {
                        const float4 v = vb[t][i4];
                        Pc[4 * i4 + 0] = fmaf(v.x, v.x, Pc[4 * i4 + 0]);
                        Pc[4 * i4 + 1] = fmaf(v.y, v.y, Pc[4 * i4 + 1]);
                        Pc[4 * i4 + 2] = fmaf(v.z, v.z, Pc[4 * i4 + 2]);
                        Pc[4 * i4 + 3] = fmaf(v.w, v.w, Pc[4 * i4 + 3]);
                    }
                }
            }
            float V[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) V[i] = Pc[i] + Pc[i + 8];
            sumsq = tree8(V[0], V[1], V[2], V[3], V[4], V[5], V[6], V[7]);
        }
        const float s = group_scale(sumsq, 1.0f / (float)GS);
        const float inv = rcp_rn(s);
        if (tg == 0) as_l[m * Kg + g] = s;
        const float4 *xc4 = reinterpret_cast<const float4 *>(xs + xpos(16 * tid));
        float4 xq[4];
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) xq[q4] = xc4[q4];
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            const float4 v = xq[q4];
            qp[m][2 * q4] = quant_pair_finite(v.x * inv, v.y * inv);
            qp[m][2 * q4 + 1] = quant_pair_finite(v.z * inv, v.w * inv);
        }
        if (__builtin_expect(!__builtin_isfinite(s), 0)) {  // a non-finite group (rare)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const float4 v = xq[q4];
                qp[m][2 * q4] = quant_pair(v.x * inv, v.y * inv);
                qp[m][2 * q4 + 1] = quant_pair(v.z * inv, v.w * inv);
            }
        }
    };
    if constexpr (P == 1) {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
#pragma unroll
            for (int j = 0; j < 8; ++j) qp[m][j] = 0;
            if (m >= M) continue;  // uniform: every thread skips together
            const float4 *src = reinterpret_cast<const float4 *>(Ap + (size_t)m * K);
            // four float4 per thread cover K/4 <= 4 * nthr (named registers; an
            // array here ends up in scratch memory)
            const int i0 = tid, i1 = tid + nthr, i2 = tid + 2 * nthr, i3 = tid + 3 * nthr;
            const float4 x0 = src[i0 < K / 4 ? i0 : 0];
            const float4 x1 = src[i1 < K / 4 ? i1 : 0];
            const float4 x2 = src[i2 < K / 4 ? i2 : 0];
            const float4 x3 = src[i3 < K / 4 ? i3 : 0];
            // fused norm: this thread's 16 weight bytes and group scale
            // (loaded unconditionally, from the activation row when there is no
            // norm, so that no later wait depends on which loads were issued)
            const int8_t *nwp = has_norm ? norm_w : reinterpret_cast<const int8_t *>(Ap);
            const float *nsp = has_norm ? norm_s : Ap;
            const u32x4 nw = *reinterpret_cast<const u32x4 *>(nwp + 16 * (act ? tid : 0));
            const float nsc = nsp[act ? (16 * tid) / GS : 0];
            if (m == 0) prefetch(resolve(tile));  // grid <= ntiles: every block has a tile
            // keep the loads above ahead of the LDS stores below (the stores wait
            // only for the activation loads, issued first); slots past K/4 exist
            // (stage_words >= 16 * nthr + padding) and are never read
            __builtin_amdgcn_sched_barrier(0);
            float4 *xs4 = reinterpret_cast<float4 *>(xs);
            xs4[xpos(4 * i0) / 4] = x0;
            xs4[xpos(4 * i1) / 4] = x1;
            xs4[xpos(4 * i2) / 4] = x2;
            xs4[xpos(4 * i3) / 4] = x3;
            if (has_norm) {
                put4(i0, x0);
                put4(i1, x1);
                put4(i2, x2);
                put4(i3, x3);
            }
            lds_barrier();
            if (has_norm) {
                norm_chain();
                lds_barrier();
                if (act) {
                    // this thread's 16 elements: x = w * ((s_g * inv) * x)
                    const float comb = nsc * s_norm_inv;
                    const uint32_t wd[4] = {nw.x, nw.y, nw.z, nw.w};
                    float4 *xc4 = reinterpret_cast<float4 *>(xs + xpos(16 * tid));
#pragma unroll
                    for (int q4 = 0; q4 < 4; ++q4) {
                        float4 v = xc4[q4];
                        const uint32_t w = wd[q4];
                        v.x = (float)(int8_t)(w & 0xFF) * (comb * v.x);
                        v.y = (float)(int8_t)((w >> 8) & 0xFF) * (comb * v.y);
                        v.z = (float)(int8_t)((w >> 16) & 0xFF) * (comb * v.z);
                        v.w = (float)(int8_t)(w >> 24) * (comb * v.w);
                        xc4[q4] = v;
                    }
                }
                lds_barrier();
            }
            if (act) quant_chunk(m);
            lds_barrier();
        }
    } else {
        // One activation row of K = 2048 over the block's 512 threads: thread
        // bt holds float4 bt, so each group of 64 elements is one row of 16
        // lanes (u = bt & 15 holds elements 4u .. 4u+3 of group bt >> 4) and
        // the group is quantized in registers, with DPP moves inside the row.
        const int bt = threadIdx.x;
        const int8_t *nwp = has_norm ? norm_w : reinterpret_cast<const int8_t *>(Ap);
        const float *nsp = has_norm ? norm_s : Ap;
        float4 xv = reinterpret_cast<const float4 *>(Ap)[bt];
        const uint32_t nw4 = *reinterpret_cast<const uint32_t *>(nwp + 4 * bt);  // norm weights of the 4
        const float nsc4 = nsp[(4 * bt) / GS];
        prefetch(resolve(tile));
        __builtin_amdgcn_sched_barrier(0);
        if (has_norm) {
            put4(bt, xv);
            lds_barrier();
            norm_chain();
            lds_barrier();
            const float comb = nsc4 * s_norm_inv;  // x = w * ((s_g * inv) * x)
            xv.x = (float)(int8_t)(nw4 & 0xFF) * (comb * xv.x);
            xv.y = (float)(int8_t)((nw4 >> 8) & 0xFF) * (comb * xv.y);
            xv.z = (float)(int8_t)((nw4 >> 16) & 0xFF) * (comb * xv.z);
            xv.w = (float)(int8_t)(nw4 >> 24) * (comb * xv.w);
        }
        // The group's sum of squares in the reference order (as the T == 4
        // quantizer): chain c = 4(u & 3) + k takes elements 16t + c, t = 0..3,
        // whose step t is lane u = 4t + (u & 3). Each round every lane extends
        // the chain value of lane u - 4 (row_shr:4; 0 into lanes 0..3), so
        // after round t lanes 4t .. 4t+3 hold chains through step t, and lanes
        // 12..15 end with the 16 chains. Then V[i] = P[i] + P[i+8] (lanes 12,
        // 13 take lanes 14, 15: row_shl:2), lane 12 takes lane 13's half
        // (row_shl:1), runs the fixed tree, and the row takes lane 12's sum
        // (row_newbcast:12).
#define Q3VL_DPPF(v, ctrl) \
    __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), ctrl, 0xF, 0xF, false))
        float c0 = fmaf(xv.x, xv.x, 0.0f), c1 = fmaf(xv.y, xv.y, 0.0f);
        float c2 = fmaf(xv.z, xv.z, 0.0f), c3 = fmaf(xv.w, xv.w, 0.0f);
#pragma unroll
        for (int t = 1; t < 4; ++t) {
            c0 = fmaf(xv.x, xv.x, Q3VL_DPPF(c0, 0x114));
            c1 = fmaf(xv.y, xv.y, Q3VL_DPPF(c1, 0x114));
            c2 = fmaf(xv.z, xv.z, Q3VL_DPPF(c2, 0x114));
            c3 = fmaf(xv.w, xv.w, Q3VL_DPPF(c3, 0x114));
        }
        const float v0 = c0 + Q3VL_DPPF(c0, 0x102), v1 = c1 + Q3VL_DPPF(c1, 0x102);
        const float v2 = c2 + Q3VL_DPPF(c2, 0x102), v3 = c3 + Q3VL_DPPF(c3, 0x102);
        const float w0 = Q3VL_DPPF(v0, 0x101), w1 = Q3VL_DPPF(v1, 0x101);
        const float w2 = Q3VL_DPPF(v2, 0x101), w3 = Q3VL_DPPF(v3, 0x101);
        const float sumsq = Q3VL_DPPF(tree8(v0, v1, v2, v3, w0, w1, w2, w3), 0x15C);
#undef Q3VL_DPPF
        const float sg = group_scale(sumsq, 1.0f / (float)GS);
        const float inv = rcp_rn(sg);
        if ((bt & 15) == 0) as_l[bt >> 4] = sg;
        uint32_t q0 = quant_pair_finite(xv.x * inv, xv.y * inv);
        uint32_t q1 = quant_pair_finite(xv.z * inv, xv.w * inv);
        if (__builtin_expect(!__builtin_isfinite(sg), 0)) {  // a non-finite group (rare)
            q0 = quant_pair(xv.x * inv, xv.y * inv);
            q1 = quant_pair(xv.z * inv, xv.w * inv);
        }
        reinterpret_cast<uint2 *>(qs)[bt] = make_uint2(q0, q1);
        lds_barrier();
        // this thread's K-chunk (float4s 4*tid .. 4*tid+3)
        const u32x4 *qs4 = reinterpret_cast<const u32x4 *>(qs) + 2 * tid;
        const u32x4 qa = qs4[0], qb = qs4[1];
        qp[0][0] = qa.x; qp[0][1] = qa.y; qp[0][2] = qa.z; qp[0][3] = qa.w;
        qp[0][4] = qb.x; qp[0][5] = qb.y; qp[0][6] = qb.z; qp[0][7] = qb.w;
    }

    // Running argmax (argmax mode) of the block's tiles, in ascending row
    // order, held by the lane that leads each activation row's chain group.
    float best = -FLT_MAX;
    int32_t bidx = -1;

    Tile cur = resolve(tile);
    for (; tile - sub < ntiles; tile += gridDim.x * P) {
        // ---- scales of the tile's rows -> LDS (values already in sv)
#pragma unroll
        for (int j = 0; j < SPT; ++j) {
            const int i = tid + j * nthr;
            const int r = i / Kg, gg = i - (i / Kg) * Kg;
            if (i < R * Kg) sc_l[r * ld + gg] = LANES ? as_l[gg] * sv[j] : sv[j];  // i8:213
        }

        // ---- phase 1: exact integer lane / group sums
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (!row_ok(cur, r)) continue;  // uniform across the block
            const uint32_t wd[4] = {wv[r].x, wv[r].y, wv[r].z, wv[r].w};
            uint32_t wp[8];
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                wp[2 * d] = lo2(wd[d]);
                wp[2 * d + 1] = hi2(wd[d]);
            }
            int32_t *Gd = seg_G(row_seg(cur, r));
            if constexpr (LANES && T <= 8) {
                // the 8 lane sums of this thread's 16 bytes, then reduced
                // over the group's T threads so that thread tg holds the
                // group totals of lanes tg*W .. tg*W + W-1 and writes them
                constexpr int W = 8 / T;
                int32_t p[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) p[j] = dot2_z(qp[0][j], wp[j]);
                scatter_sums<T>(p, tg);
                if (act) {
#pragma unroll
                    for (int k = 0; k < W; ++k) accb[(r * 8 + tg * W + k) * ld + g] = p[k] >> 8;
                }
                if (Gd) {  // the group sum: this thread's lanes, then the run's
                    int32_t tot = 0;
#pragma unroll
                    for (int k = 0; k < W; ++k) tot += p[k] >> 8;
                    tot = run_sum<T>(tot);
                    if (act && tg == 0) Gd[(size_t)row_n(cur, r) * Kg + g] = tot;
                }
            } else if constexpr (LANES) {
                int32_t p[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) p[j] = run_sum<T>(dot2_z(qp[0][j], wp[j]));
                // every thread of the group holds all 8 sums: threads 0..7
                // of the group write one each
                if (act && tg < 8) {
                    int32_t v = p[0];
#pragma unroll
                    for (int jj = 1; jj < 8; ++jj) v = jj == tg ? p[jj] : v;
                    accb[(r * 8 + tg) * ld + g] = v >> 8;
                }
                if (act && tg == 0) {
                    if (Gd) {
                        int32_t tot = 0;
#pragma unroll
                        for (int j = 0; j < 8; ++j) tot += p[j] >> 8;
                        Gd[(size_t)row_n(cur, r) * Kg + g] = tot;
                    }
                }
            } else if constexpr (T <= 8) {
                // the MR activation rows' sums, reduced over the group's T
                // threads: with MR >= T thread tg holds rows tg*W .. tg*W + W-1,
                // with MR < T the SH threads tg of row tg / SH all hold it and
                // the first writes it (rows past M carry 0 and are not written)
                constexpr int W = MR >= T ? MR / T : 1;
                constexpr int SH = MR >= T ? 1 : T / MR;
                int32_t p[MR];
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    int32_t acc = 0;
#pragma unroll
                    for (int j = 0; j < 8; ++j) acc = dot2(qp[m][j], wp[j], acc);
                    p[m] = m < M ? acc >> 8 : 0;
                }
                scatter_sums<T>(p, tg);
#pragma unroll
                for (int k = 0; k < W; ++k) {
                    const int m = (tg / SH) * W + k;
                    if (act && m < M && (SH == 1 || tg % SH == 0)) {
                        accb[(m * R + r) * ld + g] = p[k];
                        if (Gd) Gd[((size_t)m * cur.tN + row_n(cur, r)) * Kg + g] = p[k];
                    }
                }
            } else {
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    if (m >= M) break;
                    int32_t acc = 0;
#pragma unroll
                    for (int j = 0; j < 8; ++j) acc = dot2(qp[m][j], wp[j], acc);
                    acc = run_sum<T>(acc >> 8);
                    if (act && tg == 0) {
                        accb[(m * R + r) * ld + g] = acc;
                        if (Gd) Gd[((size_t)m * cur.tN + row_n(cur, r)) * Kg + g] = acc;
                    }
                }
            }
        }

        // ---- prefetch the next tile while this one finishes. (Sub-group
        // blocks issue it after the epilogue instead: there the weight stream
        // fills the memory queues, a wave issuing loads waits for queue room,
        // and that wait would hold back this tile's chains and stores.)
        const Tile t = cur;
        const int nxt = tile + gridDim.x * P;
        if (P == 1 && nxt < ntiles) {
            cur = resolve(nxt);
            prefetch(cur);
        }
        lds_barrier();

        // ---- phase 2: fp32 group chains in the reference order
        float y = 0.0f;
        int ym = 0, yr = 0;
        bool yvalid = false;
        if constexpr (LANES) {
            if (tid < 8 * R) {
                const int r = tid >> 3, j = tid & 7;
                float c = 0.0f;
                if (row_ok(t, r)) {
                    const int32_t *Lr = accb + tid * ld;
                    const float *scr = sc_l + r * ld;
                    int gg = 0;
                    // batches of 16 groups, every read of a batch issued
                    // before its FMAs
                    for (; gg + 16 <= Kg; gg += 16) {
                        int4 L4[4];
                        float4 s4[4];
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            L4[u] = *reinterpret_cast<const int4 *>(Lr + gg + 4 * u);
                            s4[u] = *reinterpret_cast<const float4 *>(scr + gg + 4 * u);
                        }
                        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            c = fmaf((float)L4[u].x, s4[u].x, c);  // i8:213-216, groups in order
                            c = fmaf((float)L4[u].y, s4[u].y, c);
                            c = fmaf((float)L4[u].z, s4[u].z, c);
                            c = fmaf((float)L4[u].w, s4[u].w, c);
                        }
                    }
                    for (; gg < Kg; ++gg) c = fmaf((float)Lr[gg], scr[gg], c);
                }
                // add_reduce_mm_256 over the row's 8 lanes (i8:219-222):
                // lane j = 0 ends with ((c0+c4) + (c1+c5)) + ((c2+c6) + (c3+c7)),
                // taking lane j+4, then j+1, then j+2 (DPP row shifts; the
                // other lanes' values are not used)
#define Q3VL_SHL(v, n) \
    __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x100 + (n), 0xF, 0xF, false))
                c = c + Q3VL_SHL(c, 4);
                c = c + Q3VL_SHL(c, 1);
                c = c + Q3VL_SHL(c, 2);
#undef Q3VL_SHL
                y = c;
                yr = r;
                yvalid = (j == 0) && row_ok(t, r);
            }
        } else {
            if (tid < M * R) {
                const int m = tid / R, r = tid - (tid / R) * R;
                float acc = 0.0f;
                if (row_ok(t, r)) {
                    const int32_t *Gr = accb + (m * R + r) * ld;
                    const float *asr = as_l + m * Kg;
                    const float *wsr = sc_l + r * ld;
                    int gg = 0;
#pragma unroll 2
                    for (; gg + 4 <= Kg; gg += 4) {
                        const int4 G4 = *reinterpret_cast<const int4 *>(Gr + gg);
                        const float4 w4 = *reinterpret_cast<const float4 *>(wsr + gg);
                        // i8:613-617 (contracted): acc = fma(G*a_s, w_s, acc)
                        acc = fmaf((float)G4.x * asr[gg + 0], w4.x, acc);
                        acc = fmaf((float)G4.y * asr[gg + 1], w4.y, acc);
                        acc = fmaf((float)G4.z * asr[gg + 2], w4.z, acc);
                        acc = fmaf((float)G4.w * asr[gg + 3], w4.w, acc);
                    }
                    for (; gg < Kg; ++gg) acc = fmaf((float)Gr[gg] * asr[gg], wsr[gg], acc);
                }
                y = acc;
                ym = m;
                yr = r;
                yvalid = row_ok(t, r);
            }
        }

        // ---- epilogues
        if (mode == GEMV_PLAIN) {
            // plain mode: every row of a tile is in segment t.tseg
            if (yvalid) {
                float *dst = seg_Y(t.tseg) + (size_t)ym * t.tN + row_n(t, yr);
                *dst = a.accumulate ? *dst + y : y;  // add_vector: to[i] += from[i]
            }
        } else if (swg) {
            if constexpr (LANES) {
                // the up row of gate row r is row r + HALF, whose sum sits
                // 8 * HALF lanes above (all in the first wave: 8R <= 64)
                const float up = __shfl_down(y, 8 * HALF);
                if (yvalid && yr < HALF) sr.Y0[row_n(t, yr)] = silu_mul(y, up);
            } else {
                if (yvalid) ybuf[ym * R + yr] = y;
                lds_barrier();
                if (tid < M * HALF) {
                    const int m = tid / HALF, r = tid - (tid / HALF) * HALF;
                    if (row_ok(t, r))
                        sr.Y0[(size_t)m * t.tN + row_n(t, r)] =
                            silu_mul(ybuf[m * R + r], ybuf[m * R + r + HALF]);
                }
            }
        } else {  // GEMV_ARGMAX, in registers of the wave that holds y
            if (yvalid && sr.Y0) sr.Y0[(size_t)ym * t.tN + row_n(t, yr)] = y;
            // candidate: a valid row whose value beats -FLT_MAX (NaN never)
            float cv = y;
            int32_t ci = (yvalid && y > -FLT_MAX) ? row_n(t, yr) : -1;
            // The tile's rows of one activation row sit in R lanes spaced by
            // RS (lanes: rows are 8 lanes apart; general: adjacent lanes).
            constexpr int RS = LANES ? 8 : 1;
#pragma unroll
            for (int off = RS; off < RS * R; off <<= 1) {
                const float ov = __shfl_xor(cv, off);
                const int32_t oi = __shfl_xor(ci, off);
                am_combine(cv, ci, ov, oi);  // larger value, then lower index
            }
            // Rows of later tiles have larger indices: a strict > keeps the
            // first occurrence, as greedy_decode's scan does.
            if (tid < M * R * RS && (tid & (RS * R - 1)) == 0 && ci >= 0 &&
                (bidx < 0 || cv > best)) {
                best = cv;
                bidx = ci;
            }
        }
        if (P > 1 && nxt - sub < ntiles) {
            cur = resolve(nxt);
            prefetch(cur);
        }
        lds_barrier();
    }

    if (mode != GEMV_ARGMAX) return;
    // ---- argmax: this block's (value, index) partial per activation row, in
    // its own slots (no shared counters or atomics: 2048 blocks contending on
    // one address serialize); argmax_final_kernel reduces the partials.
    // The running best of activation row m lives on lane m*R (general) or
    // lane 0 (lanes, M == 1).
    const int lead = LANES ? 0 : (tid % R == 0 && tid < M * R ? tid / R : -1);
    if constexpr (P > 1) {  // one activation row: the sub-groups' lane 0, combined
        __shared__ float sbv[P];
        __shared__ int32_t sbi[P];
        if (tid == 0) {
            sbv[sub] = best;
            sbi[sub] = bidx;
        }
        lds_barrier();
        if (threadIdx.x == 0) {
            for (int q = 1; q < P; ++q) am_combine(best, bidx, sbv[q], sbi[q]);
            a.part_val[blockIdx.x] = best;
            a.part_idx[blockIdx.x] = bidx;
        }
    } else if ((LANES ? tid == 0 : lead >= 0)) {
        const int m = LANES ? 0 : lead;
        a.part_val[(size_t)blockIdx.x * M + m] = best;
        a.part_idx[(size_t)blockIdx.x * M + m] = bidx;
    }
}

// ------------------------------------------------------ streaming decode GEMV
// The decode step's lane-path launches (one activation row, group 64, K = KC
// of 2048 or 6144; plain / accumulate over up to three segments, or gate|up
// with the SwiGLU epilogue; the fused RMSNorm at K = 2048), in the same
// reference order as gemv_kernel, with each row tile one wave's work.
//
// Prologue (once per block): the activation row is normalized (fused norm)
// and quantized, 8 lanes per group, into LDS; one block barrier. After it
// every wave walks its own row tiles (R rows each, stride gridDim.x*NW) with
// no block barrier. A tile's R*Kg (row, group) pairs are taken 64 at a time
// ("passes"), one per lane: the lane loads the group's 64 weight bytes (four
// 16-byte loads) and accumulates the 8 exact int32 lane sums of the group
// (i8:188-211) with v_dot2 -- no cross-lane reduction -- and writes them as
// floats, with the combined scale fl(a_s * w_s), to the wave's own LDS rows.
// Then lanes 8r + j run row r's fp32 chains over the groups (i8:213-216) and
// the 8-lane tree (i8:219-222). The next tile's weights and scales are loaded
// before this tile's phases.
template <int KC, int MD, int R, int NW>
__global__ __launch_bounds__(64 * NW) void gemv_stream_kernel(
    const int8_t *W0, const int8_t *W1, const int8_t *W2, const float *S0, const float *S1,
    const float *S2, int N0, int N1, GemvArgs a, int ntiles) {
    constexpr int GS = 64, NTH = 64 * NW;
    constexpr int K = KC, Kg = K / GS;
    constexpr int CPL = K / 1024;            // K-chunks per lane and weight row
    constexpr int SPL = (R * Kg + 63) / 64;  // weight scales per lane and tile
    constexpr int HALF = R / 2;
    constexpr bool SWG = MD == MD_SWIGLU;
    constexpr int LD = (((Kg + 3) & ~3) >> 2) & 1 ? ((Kg + 3) & ~3) : ((Kg + 3) & ~3) + 4;  // group_ld(Kg)
    constexpr int QLD = 36;  // words per group of the quantized row (32 + 4 padding)
    constexpr bool SEGN = norm_seg(KC);
    constexpr int NRS = norm_row_words(K, SEGN);
    static_assert(KC == 2048 || KC == 6144, "decode row lengths");
    static_assert(8 * R <= 64, "a tile's chains fit one wave");
    static_assert(!SWG || R % 2 == 0, "gate and up rows in pairs");
    static_assert(MD == MD_SWIGLU || MD == MD_RUNTIME, "plain or swiglu");
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ float s_norm_inv;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    // LDS: the quantized row ([Kg][QLD] words), a_s, the fused norm's
    // chain-major copy (K = 2048), then per wave its lane sums [8R][LD] and
    // combined scales [R][LD]
    uint32_t *qs = reinterpret_cast<uint32_t *>(smem);
    float *as_l = reinterpret_cast<float *>(qs + Kg * QLD);
    float *xn = as_l + ((Kg + 3) & ~3);
    float *accb = xn + (KC == 2048 ? 8 * NRS : 0) + wid * (9 * R * LD);
    float *scb = accb + 8 * R * LD;
    const bool has_norm = KC == 2048 && a.norm_w != nullptr;

    SegRegs sr;
    sr.W0 = W0; sr.W1 = W1; sr.W2 = W2;
    sr.S0 = S0; sr.S1 = S1; sr.S2 = S2;
    sr.Y0 = a.seg[0].Y; sr.Y1 = a.seg[1].Y; sr.Y2 = a.seg[2].Y;
    sr.N0 = N0; sr.N1 = N1; sr.N2 = a.seg[2].N;
    int nseg = SWG ? 2 : a.nseg;
    asm volatile("" : "+s"(sr.N0), "+s"(sr.N1), "+s"(sr.N2));
    if constexpr (!SWG) asm volatile("" : "+s"(nseg));
    sr.t1 = (sr.N0 + R - 1) / R;
    sr.t2 = nseg > 2 ? sr.t1 + (sr.N1 + R - 1) / R : 0x7fffffff;
    if (SWG || nseg < 2) sr.t1 = 0x7fffffff;
    auto resolve = [&](int tile) {
        Tile t;
        if constexpr (SWG) {
            t.tseg = 0;
            t.tn0 = tile * HALF;
            t.tN = sr.N0;
        } else {
            t.tseg = tile < sr.t1 ? 0 : (tile < sr.t2 ? 1 : 2);
            t.tn0 = (tile - pick3(t.tseg, 0, sr.t1, sr.t2)) * R;
            t.tN = pick3(t.tseg, sr.N0, sr.N1, sr.N2);
        }
        return t;
    };
    auto row_seg = [&](const Tile &t, int r) { return SWG ? (r < HALF ? 0 : 1) : t.tseg; };
    auto row_n = [&](const Tile &t, int r) { return SWG ? t.tn0 + r % (HALF > 0 ? HALF : 1) : t.tn0 + r; };
    auto row_ok = [&](const Tile &t, int r) { return row_n(t, r) < t.tN; };

    // ---- one tile's weight chunks and scales into registers. Rows past the
    // segment end read row 0 (the value is never used: no select on loaded
    // data, so nothing waits at issue). Scales first: the scale products at
    // the top of a tile then wait only for them (loads retire in order).
    u32x4 wv[2][R][CPL];
    float sv[2][SPL];
    auto load_tile = [&](auto B, const Tile &t) {
        constexpr int b = decltype(B)::value;
#pragma unroll
        for (int s = 0; s < SPL; ++s) {
            const int e = lane + 64 * s, r = e / Kg, gg = e % Kg;
            const bool ok = r < R && row_ok(t, r);
            const float *S = pick3(row_seg(t, r < R ? r : 0), sr.S0, sr.S1, sr.S2);
            sv[b][s] = S[ok ? (size_t)row_n(t, r) * Kg + gg : 0];
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int8_t *w = pick3(row_seg(t, r), sr.W0, sr.W1, sr.W2) +
                              (size_t)(row_ok(t, r) ? row_n(t, r) : 0) * K;
#pragma unroll
            for (int i = 0; i < CPL; ++i)
                wv[b][r][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(w) + lane + 64 * i);
        }
    };

    int tile = blockIdx.x * NW + wid;
    const int stride = gridDim.x * NW;
    // (a wave with no tile loads the last one, unused: no branch around loads)
    Tile cur = resolve(tile < ntiles ? tile : ntiles - 1);

    // ---- phase 0 (i8:135-177): the group quantizer, 8 lanes a group. Lane
    // u of group g holds elements 64g + 16t + 2u + k (t = 0..3, k = 0, 1),
    // i.e. chains 2u and 2u + 1 of the group's 16 sum-of-squares chains
    // (chain c takes elements 16t + c in ascending t). Its loads are issued
    // before the first tile's weight loads, so waiting for them does not wait
    // for the weights.
    constexpr int QIT = (8 * Kg + NTH - 1) / NTH;  // quantizer passes (whole waves)
    float2 xq[QIT][4];
    uint32_t nwq[QIT][4];
    float nsq[QIT];
#pragma unroll
    for (int it = 0; it < QIT; ++it) {
        const int qi = tid + NTH * it;
        if (qi < 8 * Kg) {  // wave-uniform
            const int g = qi >> 3, u = qi & 7;
            const float *xg = a.A + 64 * g + 2 * u;
#pragma unroll
            for (int t = 0; t < 4; ++t) xq[it][t] = *reinterpret_cast<const float2 *>(xg + 16 * t);
            if (has_norm) {
                const int8_t *nw = a.norm_w + 64 * g + 2 * u;
#pragma unroll
                for (int t = 0; t < 4; ++t) nwq[it][t] = *reinterpret_cast<const uint16_t *>(nw + 16 * t);
                nsq[it] = a.norm_s[g];
            }
        }
    }
    load_tile(std::integral_constant<int, 0>{}, cur);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (KC == 2048) {
        static_assert(KC != 2048 || QIT == 1, "one quantizer pass at K = 2048");
        if (has_norm) {
            // the fused norm's inverse rms: the row into the chain-major copy
            // (element e in chain e % 8 at e / 8), then the 8-chain sum of
            // squares
            if (tid < 8 * Kg) {
                const int g = tid >> 3, u = tid & 7;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
#pragma unroll
                    for (int k = 0; k < 2; ++k) {
                        const int l = (2 * u + k) & 7;
                        const int pos = 8 * g + 2 * t + ((2 * u + k) >> 3);
                        xn[l * NRS + (SEGN ? pos + 4 * (pos >> 5) : pos)] = k ? xq[0][t].y : xq[0][t].x;
                    }
                }
            }
            lds_barrier();
            if (tid < 64) {
                // The sum of squares in the reference's 8-lane order: lane
                // 8l + j holds segment j (positions 32j .. 32j+31) of chain l;
                // in segment s only lanes j == s carry their chain, and a row
                // shift hands each chain's sum to its next segment's lane.
                const float *sg = xn + (tid >> 3) * NRS + (tid & 7) * 36;
                float4 X[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) X[u] = reinterpret_cast<const float4 *>(sg)[u];
                float acc = 0.0f;
#pragma unroll
                for (int sgm = 0; sgm < 8; ++sgm) {
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        acc = fmaf(X[u].x, X[u].x, acc);
                        acc = fmaf(X[u].y, X[u].y, acc);
                        acc = fmaf(X[u].z, X[u].z, acc);
                        acc = fmaf(X[u].w, X[u].w, acc);
                    }
                    if (sgm < 7)  // row_shr:1
                        acc = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                  0, __builtin_bit_cast(int, acc), 0x111, 0xF, 0xF, false));
                }
                // chain l's sum sits in lane 8l + 7; added in chain order
                float ss = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), 7));
#pragma unroll
                for (int l = 1; l < 8; ++l)
                    ss = ss + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), 8 * l + 7));
                if (tid == 0) s_norm_inv = rcp_rn(sqrt_rn(ss * rcp_rn((float)K) + a.norm_eps));
            }
            lds_barrier();
            if (tid < 8 * Kg) {
                const float comb = nsq[0] * s_norm_inv;  // x = w * ((s_g * inv) * x)
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    xq[0][t].x = (float)(int8_t)(nwq[0][t] & 0xFF) * (comb * xq[0][t].x);
                    xq[0][t].y = (float)(int8_t)(nwq[0][t] >> 8) * (comb * xq[0][t].y);
                }
            }
        }
    }
    // The quantizer proper. V[i] = P[i] + P[i+8] (lane u < 4 takes lane u + 4:
    // row_shl:4), then the fixed tree ((V0+V4)+(V1+V5)) + ((V2+V6)+(V3+V7))
    // over lanes 0..3 (row_shl:2, row_shl:1), broadcast from the group's
    // lane 0.
#define Q3VL_DPPF(v, ctrl) \
    __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), ctrl, 0xF, 0xF, false))
#pragma unroll
    for (int it = 0; it < QIT; ++it) {
        const int qi = tid + NTH * it;
        if (qi >= 8 * Kg) break;  // wave-uniform
        const int g = qi >> 3, u = qi & 7;
        const float2 *xv = xq[it];
        float c0 = fmaf(xv[0].x, xv[0].x, 0.0f), c1 = fmaf(xv[0].y, xv[0].y, 0.0f);
#pragma unroll
        for (int t = 1; t < 4; ++t) {
            c0 = fmaf(xv[t].x, xv[t].x, c0);
            c1 = fmaf(xv[t].y, xv[t].y, c1);
        }
        const float s0 = c0 + Q3VL_DPPF(c0, 0x104), s1 = c1 + Q3VL_DPPF(c1, 0x104);
        const float y0 = s0 + Q3VL_DPPF(s0, 0x102), y1 = s1 + Q3VL_DPPF(s1, 0x102);
        const float z = y0 + y1;
        const float sum = z + Q3VL_DPPF(z, 0x101);
        // lane 0 of the quad to the quad, then lanes 4..7 take lanes 0..3
        // (row_shr:4 on banks 1 and 3 only)
        const int b0 = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sum), 0x00, 0xF, 0xF, false);
        const float sumsq = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(b0, b0, 0x114, 0xF, 0xA, false));
        const float sg = group_scale(sumsq, 1.0f / (float)GS);
        const float inv = rcp_rn(sg);
        if (u == 0) as_l[g] = sg;
        uint32_t q[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) q[t] = quant_pair_finite(xv[t].x * inv, xv[t].y * inv);
        if (__builtin_expect(!__builtin_isfinite(sg), 0)) {  // a non-finite group (rare)
#pragma unroll
            for (int t = 0; t < 4; ++t) q[t] = quant_pair(xv[t].x * inv, xv[t].y * inv);
        }
        // pair 8t + u of the group
#pragma unroll
        for (int t = 0; t < 4; ++t) qs[QLD * g + 8 * t + u] = q[t];
    }
#undef Q3VL_DPPF
    lds_barrier();

    // this lane's K-chunks of the quantized row (8 int16 pairs each) and the
    // a_s of its scale elements
    uint32_t qp[CPL][8];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int ch = lane + 64 * i;  // K-chunk: group ch / 4, pairs 8 (ch % 4) ..
        const u32x4 *q4 = reinterpret_cast<const u32x4 *>(qs + QLD * (ch >> 2) + 8 * (ch & 3));
        const u32x4 qa = q4[0], qb = q4[1];
        qp[i][0] = qa.x; qp[i][1] = qa.y; qp[i][2] = qa.z; qp[i][3] = qa.w;
        qp[i][4] = qb.x; qp[i][5] = qb.y; qp[i][6] = qb.z; qp[i][7] = qb.w;
    }
    float asv[SPL];
#pragma unroll
    for (int s = 0; s < SPL; ++s) asv[s] = as_l[(lane + 64 * s) % Kg];

    const int tg = lane & 3;
    const int cr = lane >> 3;  // the chain lane's row (lane 8r + j)
    // One tile from buffer B; the next tile's loads go to the other buffer
    // first. Returns false when the wave has no further tile.
    auto step = [&](auto B) -> bool {
        constexpr int b = decltype(B)::value;
        const Tile t = cur;
        const int nxt = tile + stride;
        if (nxt < ntiles) {  // wave-uniform
            cur = resolve(nxt);
            load_tile(std::integral_constant<int, b ^ 1>{}, cur);
        }
        // ---- the combined scales fl(a_s * w_s) of the tile's rows (i8:213)
#pragma unroll
        for (int s = 0; s < SPL; ++s) {
            const int e = lane + 64 * s, r = e / Kg, gg = e % Kg;
            if (r < R) scb[r * LD + gg] = asv[s] * sv[b][s];
        }
        // ---- phase 1: the exact int32 lane sums of every group: the 8 lane
        // partials of this lane's 16 bytes (weights in the high bytes: 256x),
        // reduce-scattered over the group's lane quad; lane tg writes lanes
        // 2tg and 2tg+1 of the group
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const u32x4 w4 = wv[b][r][i];
                const uint32_t wd[4] = {w4.x, w4.y, w4.z, w4.w};
                int32_t p[8];
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    p[2 * d] = dot2_z(qp[i][2 * d], lo2(wd[d]));
                    p[2 * d + 1] = dot2_z(qp[i][2 * d + 1], hi2(wd[d]));
                }
                scatter_sums<4>(p, tg);
                const int g = (lane + 64 * i) >> 2;
                accb[(r * 8 + 2 * tg) * LD + g] = (float)(p[0] >> 8);
                accb[(r * 8 + 2 * tg + 1) * LD + g] = (float)(p[1] >> 8);
            }
        }
        // (LDS operations of one wave complete in order: the reads below see
        // the writes above without a barrier)
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        // ---- phase 2: lane 8r + j runs row r's chain over the groups in
        // ascending order (i8:213-216)
        float c = 0.0f;
        if (lane < 8 * R) {
            const float *Lr = accb + lane * LD;
            const float *scr = scb + cr * LD;
#pragma unroll
            for (int gg = 0; gg < Kg; gg += 16) {
                float4 L4[4], s4[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    L4[u] = *reinterpret_cast<const float4 *>(Lr + gg + 4 * u);
                    s4[u] = *reinterpret_cast<const float4 *>(scr + gg + 4 * u);
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    c = fmaf(L4[u].x, s4[u].x, c);
                    c = fmaf(L4[u].y, s4[u].y, c);
                    c = fmaf(L4[u].z, s4[u].z, c);
                    c = fmaf(L4[u].w, s4[u].w, c);
                }
            }
        }
        // add_reduce_mm_256 over the row's 8 lanes (i8:219-222): lane j = 0
        // ends with ((c0+c4) + (c1+c5)) + ((c2+c6) + (c3+c7))
#define Q3VL_SHL(v, n) \
    __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x100 + (n), 0xF, 0xF, false))
        c = c + Q3VL_SHL(c, 4);
        c = c + Q3VL_SHL(c, 1);
        c = c + Q3VL_SHL(c, 2);
#undef Q3VL_SHL
        // ---- epilogue
        const bool yvalid = lane < 8 * R && (lane & 7) == 0 && row_ok(t, cr);
        if constexpr (SWG) {
            // the up row of gate row r is row r + HALF, 8 * HALF lanes above
            const float up = __shfl_down(c, 8 * HALF);
            if (yvalid && cr < HALF) sr.Y0[row_n(t, cr)] = silu_mul(c, up);
        } else {
            if (yvalid) {
                float *dst = pick3(t.tseg, sr.Y0, sr.Y1, sr.Y2) + row_n(t, cr);
                *dst = a.accumulate ? *dst + c : c;  // add_vector: to[i] += from[i]
            }
        }
        // the next tile rewrites this wave's LDS rows after the reads above
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        tile = nxt;
        return nxt < ntiles;
    };
    if (tile < ntiles) {
        while (step(std::integral_constant<int, 0>{}) && step(std::integral_constant<int, 1>{})) {
        }
    }
}

__device__ void am_block_reduce(float &bv, int32_t &bi) {
    __shared__ float sv[256];
    __shared__ int32_t si[256];
    const int tid = threadIdx.x;
    sv[tid] = bv;
    si[tid] = bi;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (tid < w) {
            float v = sv[tid];
            int32_t i = si[tid];
            am_combine(v, i, sv[tid + w], si[tid + w]);
            sv[tid] = v;
            si[tid] = i;
        }
        __syncthreads();
    }
    bv = sv[0];
    bi = si[0];
    __syncthreads();
}

// Reduces block partials [nparts, M] to ids[m] (empty partials have idx < 0;
// none at all -> 0, as greedy_decode returns 0 when nothing beats -FLT_MAX).
// One 256-thread block per row m: each thread issues all of its loads of a
// pass (8 partials, indices clamped into the buffer, so every load is
// unconditional) before combining them, then each wave reduces by DPP moves
// (quad swaps and row mirrors, then the four rows' lane 0) and lane 0 of
// wave 0 combines the four waves. The combine (larger value, then lower
// index, empties ignored) selects one element of a total order, so any
// reduction order gives the same (value, index).
__global__ __launch_bounds__(256) void argmax_final_kernel(const float *pv, const int32_t *pi,
                                                           int nparts, int M, int32_t *ids,
                                                           int32_t *pos_inc) {
    __shared__ float wv[4];
    __shared__ int32_t wi[4];
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int m = blockIdx.x;
    float bv = -FLT_MAX;
    int32_t bi = -1;
    for (int p0 = 0; p0 < nparts; p0 += 8 * 256) {
        float v[8];
        int32_t ix[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int p = p0 + tid + u * 256;
            const size_t at = (size_t)min(p, nparts - 1) * M + m;
            v[u] = pv[at];
            ix[u] = pi[at];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) am_combine(bv, bi, v[u], p0 + tid + u * 256 < nparts ? ix[u] : -1);
    }
#define Q3VL_DPPV(x, ctrl) \
    __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), ctrl, 0xF, 0xF, false))
#define Q3VL_DPPI(x, ctrl) __builtin_amdgcn_mov_dpp(x, ctrl, 0xF, 0xF, false)
    // quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror: every lane
    // of a row of 16 ends with the row's combine
    {
        float ov = Q3VL_DPPV(bv, 0xB1);
        int32_t oi = Q3VL_DPPI(bi, 0xB1);
        am_combine(bv, bi, ov, oi);
        ov = Q3VL_DPPV(bv, 0x4E);
        oi = Q3VL_DPPI(bi, 0x4E);
        am_combine(bv, bi, ov, oi);
        ov = Q3VL_DPPV(bv, 0x141);
        oi = Q3VL_DPPI(bi, 0x141);
        am_combine(bv, bi, ov, oi);
        ov = Q3VL_DPPV(bv, 0x140);
        oi = Q3VL_DPPI(bi, 0x140);
        am_combine(bv, bi, ov, oi);
    }
#undef Q3VL_DPPV
#undef Q3VL_DPPI
    auto rdv = [&](int l) {
        return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, bv), l));
    };
    float rv = rdv(0);
    int32_t ri = __builtin_amdgcn_readlane(bi, 0);
#pragma unroll
    for (int r = 1; r < 4; ++r) am_combine(rv, ri, rdv(16 * r), __builtin_amdgcn_readlane(bi, 16 * r));
    if (lane == 0) {
        wv[wid] = rv;
        wi[wid] = ri;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 4; ++w) am_combine(rv, ri, wv[w], wi[w]);
        ids[m] = ri < 0 ? 0 : ri;
        if (pos_inc && m == 0) *pos_inc += 1;
    }
}

// Stand-alone argmax over logits rows: block b scans a contiguous slice with
// the strict > rule, emitting (value, index) partials in [nparts, M] layout.
__global__ __launch_bounds__(256) void argmax_part_kernel(const float *logits, int M, int V,
                                                          int nparts, float *pv, int32_t *pi) {
    const int m = blockIdx.y;
    const int per = (V + nparts - 1) / nparts;
    const int lo = blockIdx.x * per;
    const int hi = min(V, lo + per);
    float bv = -FLT_MAX;
    int32_t bi = -1;
    for (int i = lo + threadIdx.x; i < hi; i += blockDim.x) {
        const float v = logits[(size_t)m * V + i];
        if (v > -FLT_MAX) am_combine(bv, bi, v, i);
    }
    am_block_reduce(bv, bi);
    if (threadIdx.x == 0) {
        pv[(size_t)blockIdx.x * M + m] = bv;
        pi[(size_t)blockIdx.x * M + m] = bi;
    }
}

__global__ void swiglu_kernel(float *gate, const float *up, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) gate[i] = silu_mul(gate[i], up[i]);
}

// ------------------------------------------------------------------ launch
// Launch-size cache of one kernel instantiation: the full-occupancy grid
// (CUs x resident blocks) per (device, threads, LDS bytes).
struct GridCache {
    struct Entry {
        int dev, nthr;
        size_t lds;
        int grid;
    };
    std::mutex mu;
    std::vector<Entry> entries;
    int find(int dev, int nthr, size_t lds) {
        std::lock_guard<std::mutex> lk(mu);
        for (const Entry &x : entries)
            if (x.dev == dev && x.nthr == nthr && x.lds == lds) return x.grid;
        return 0;
    }
    void put(int dev, int nthr, size_t lds, int grid) {
        std::lock_guard<std::mutex> lk(mu);
        entries.push_back({dev, nthr, lds, grid});
    }
};

// CU count per device, queried once.
static hipError_t device_cus(int dev, int *cus) {
    static std::mutex mu;
    static std::vector<int> known;  // index: device, 0 = not queried
    std::lock_guard<std::mutex> lk(mu);
    if (dev >= (int)known.size()) known.resize(dev + 1, 0);
    if (known[dev] <= 0) {
        int n = 0;
        hipError_t e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return e;
        known[dev] = n < 1 ? 1 : n;
    }
    *cus = known[dev];
    return hipSuccess;
}

template <int GS, int MR, bool LANES, int R, int KC = 0, int MD = MD_RUNTIME, int P = 1>
static hipError_t launch_gemv_t(const GemvArgs &a, int *grid_out, hipStream_t st) {
    const int K = a.K, Kg = K / GS;
    const int nthr = K / 16 > 64 ? K / 16 : 64;
    if (P > 1 && (K != KC || a.M != 1)) return hipErrorInvalidValue;
    const int ld = group_ld(Kg);
    const int acc_words = (LANES ? 8 * R : MR * R) * ld;
    const int stage_need = 16 * nthr + 4 * (16 * nthr / GS) +
                           (a.norm_w ? 8 * norm_row_words(K, norm_seg(KC)) : 0);
    const int stage_words = P * acc_words > stage_need ? P * acc_words : stage_need;
    const size_t lds =
        (size_t)(stage_words + MR * Kg + (P > 1 ? 8 * nthr : 0) + P * (R * ld + MR * R)) * 4;

    int ntiles = 0;
    if (a.mode == GEMV_SWIGLU) {
        ntiles = (a.seg[0].N + R / 2 - 1) / (R / 2);
    } else {
        for (int s = 0; s < a.nseg; ++s) ntiles += (a.seg[s].N + R - 1) / R;
    }
    // CUs x resident blocks per CU of this instantiation, queried once per
    // (device, threads, LDS bytes) and then looked up
    static GridCache cache;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    int grid = cache.find(dev, P * nthr, lds);
    if (grid <= 0) {
        int cus = 0, occ = 0;
        e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return e;
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, gemv_kernel<GS, MR, LANES, R, KC, MD, P>,
                                                         P * nthr, lds);
        if (e != hipSuccess) return e;
        grid = cus * (occ < 1 ? 1 : occ);
        cache.put(dev, P * nthr, lds, grid);
    }
    if (grid > GEMV_MAX_GRID) grid = GEMV_MAX_GRID;  // argmax partials reserved per launch
    if (grid > (ntiles + P - 1) / P) grid = (ntiles + P - 1) / P;
    if (grid < 1) grid = 1;
    if (grid_out) *grid_out = grid;
    gemv_kernel<GS, MR, LANES, R, KC, MD, P><<<grid, P * nthr, lds, st>>>(
        a.seg[0].W, a.seg[1].W, a.seg[2].W, a.seg[0].S, a.seg[1].S, a.seg[2].S, a.seg[0].N,
        a.seg[1].N, a, ntiles);
    return hipGetLastError();
}

// Rows per tile of the M = 1 lane path: the largest of 8, 4, 2 that still
// gives about four tiles per CU. Small GEMVs (one tile per block) are bound by
// the latency of each block's dependent phases, so more and smaller blocks
// let those phases overlap across waves; each block repeats the activation
// quantization, which grows with K, so long rows (K > 4096) keep 8 rows.
static int lane_rows(const GemvArgs &a) {
    if (a.K > 4096) return 8;
    auto tiles = [&](int r) {
        if (a.mode == GEMV_SWIGLU) return (a.seg[0].N + r / 2 - 1) / (r / 2);
        int t = 0;
        for (int s = 0; s < a.nseg; ++s) t += (a.seg[s].N + r - 1) / r;
        return t;
    };
    if (tiles(8) >= 1024) return 8;
    if (tiles(4) >= 1024) return 4;
    return 2;
}

// The lane path with K fixed at compile time for the decode step's row
// lengths at group size 64.
template <int GS, int R, int KC, int P = 1>
static hipError_t launch_lanes_k(const GemvArgs &a, int *grid_out, hipStream_t st) {
    if (a.mode == GEMV_SWIGLU && a.nseg == 2) return launch_gemv_t<GS, 1, true, R, KC, MD_SWIGLU, P>(a, grid_out, st);
    if (a.mode == GEMV_ARGMAX && a.nseg == 1) return launch_gemv_t<GS, 1, true, R, KC, MD_ARGMAX1, P>(a, grid_out, st);
    return launch_gemv_t<GS, 1, true, R, KC, MD_RUNTIME, P>(a, grid_out, st);
}

template <int GS, int R, int P = 1>
static hipError_t launch_lanes(const GemvArgs &a, int *grid_out, hipStream_t st) {
    if constexpr (GS == 64) {
        if (a.K == 2048) return launch_lanes_k<GS, R, 2048, P>(a, grid_out, st);
        if (a.K == 6144) return launch_lanes_k<GS, R, 6144>(a, grid_out, st);
    }
    return launch_gemv_t<GS, 1, true, R>(a, grid_out, st);
}

// Rows per tile when blocks work on kSubGroups tiles side by side (K = 2048,
// group 64): the tile groups should spread evenly over the CUs, since a CU
// left with one group more than the others sets the kernel's length. Of
// 8, 4 and 2 rows, the largest whose rounding waste (group slots left idle
// in the last round over the CUs) is within 5% of the smallest. Returns 0
// when that leaves more than 4 groups per CU: blocks that loop over many
// tiles are held back by the block-wide barriers between their tiles (the
// sub-groups wait for each other's weights), and run one tile per block
// instead. Measured at the decode shapes: q|k|v 4 rows (256 groups), o 2
// (256), gate|up 4 (768) are 2-14% faster than one tile per block; lm_head
// (4748 groups) was 14% slower inside the decode step.
static int lane_rows_sub(const GemvArgs &a, int cus) {
    auto tiles = [&](int r) {
        if (a.mode == GEMV_SWIGLU) return (a.seg[0].N + r / 2 - 1) / (r / 2);
        int t = 0;
        for (int s = 0; s < a.nseg; ++s) t += (a.seg[s].N + r - 1) / r;
        return t;
    };
    double waste[3];
    const int rows[3] = {8, 4, 2};
    double best = 1.0;
    for (int i = 0; i < 3; ++i) {
        const int groups = (tiles(rows[i]) + kSubGroups - 1) / kSubGroups;
        const int slots = (groups + cus - 1) / cus * cus;
        waste[i] = (double)(slots - groups) / slots;
        best = waste[i] < best ? waste[i] : best;
    }
    for (int i = 0; i < 3; ++i) {
        if (waste[i] <= best + 0.05) {
            const int groups = (tiles(rows[i]) + kSubGroups - 1) / kSubGroups;
            return groups > 4 * cus ? 0 : rows[i];
        }
    }
    return 0;
}


// ---- the streaming decode GEMV's launch
struct StreamCfg {
    int nw, r;  // waves per block, rows per wave tile (0: not taken)
    int bpc;    // blocks per CU at most, 0: one tile per wave (else the waves loop over tiles)
};

// Measured at the decode shapes (MI355X, us per launch: a HIP graph of one
// launch per weight copy, with more than 640 MB of copies so that every
// launch streams its weights from HBM, as in the decode step; gemv_kernel's
// in brackets):
//   q|k|v   K = 2048, 4096 rows:  8 waves, 2 rows, 256 blocks      4.11 (4.38)
//   o       K = 2048, 2048 rows:  8 waves, 1 row, 256 blocks       3.26 (3.42)
//   gate|up K = 2048, 2 x 6144:   4 waves, 2+2 rows, 768 blocks    7.39 (7.61)
//   down    K = 6144, 2048 rows:  8 waves, 1 row, 256 blocks       5.37 (6.34)
// Plain reads of the same bytes from HBM in the same replay take 2.2 (4 MB),
// 2.8 (8 MB), 3.8 (12 MB) and 5.4 us (24 MB); an empty kernel 2.2 us.
static StreamCfg stream_cfg(const GemvArgs &a) {
    if (a.mode == GEMV_SWIGLU) return {4, 4, 0};
    if (a.K == 6144) return {8, 1, 0};
    int rows = 0;
    for (int s = 0; s < a.nseg; ++s) rows += a.seg[s].N;
    if (rows <= 2048) return {8, 1, 0};
    // 3-row tiles where 2-row tiles would need more than one 8-wave block
    // per CU and 3-row tiles need at most one (6144 rows: 256 blocks instead
    // of 384, half the CUs holding two; graph replay from HBM 5.2 -> 4.9 us)
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) == hipSuccess && device_cus(dev, &cus) == hipSuccess && a.nseg == 1 &&
        (rows + 15) / 16 > cus && (rows + 23) / 24 <= cus)
        return {8, 3, 0};
    return {8, 2, 0};
}

static size_t stream_lds(int KC, int R, int NW) {
    const int Kg = KC / 64, ld = group_ld(Kg);
    return (size_t)4 * (36 * Kg + ((Kg + 3) & ~3) + (KC == 2048 ? 8 * norm_row_words(KC, norm_seg(KC)) : 0) +
                        NW * 9 * R * ld);
}

template <int KC, int MD, int R, int NW>
static hipError_t launch_stream_t(const GemvArgs &a, int bpc, int *grid_out, hipStream_t st) {
    int ntiles = 0;
    if (MD == MD_SWIGLU) {
        ntiles = (a.seg[0].N + R / 2 - 1) / (R / 2);
    } else {
        for (int s = 0; s < a.nseg; ++s) ntiles += (a.seg[s].N + R - 1) / R;
    }
    if (ntiles < 1) return hipSuccess;
    int dev = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = device_cus(dev, &cus);
    if (e != hipSuccess) return e;
    int grid = (ntiles + NW - 1) / NW;
    if (bpc > 0 && grid > bpc * cus) grid = bpc * cus;
    if (grid_out) *grid_out = grid;
    // (K = 6144 with 8 waves of 2 rows needs more than the default 64 KiB)
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void *>(&gemv_stream_kernel<KC, MD, R, NW>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)stream_lds(KC, R, NW));
    if (attr != hipSuccess) return attr;
    gemv_stream_kernel<KC, MD, R, NW><<<grid, 64 * NW, stream_lds(KC, R, NW), st>>>(
        a.seg[0].W, a.seg[1].W, a.seg[2].W, a.seg[0].S, a.seg[1].S, a.seg[2].S, a.seg[0].N, a.seg[1].N, a,
        ntiles);
    return hipGetLastError();
}

template <int KC, int MD>
static hipError_t launch_stream_md(const GemvArgs &a, const StreamCfg &c, int *grid_out, hipStream_t st) {
#define Q3VL_STREAM(R_, NW_) \
    if (c.r == R_ && c.nw == NW_) return launch_stream_t<KC, MD, R_, NW_>(a, c.bpc, grid_out, st);
    if constexpr (MD != MD_SWIGLU) {
        Q3VL_STREAM(1, 4)
        Q3VL_STREAM(1, 8)
        if constexpr (KC == 2048) Q3VL_STREAM(3, 8)
    }
    Q3VL_STREAM(2, 4)
    Q3VL_STREAM(2, 8)
    if constexpr (KC == 2048) {  // (4 rows of 6144 bytes, double-buffered, exceed the registers)
        Q3VL_STREAM(4, 4)
        Q3VL_STREAM(4, 8)
    }
#undef Q3VL_STREAM
    return hipErrorInvalidValue;
}

// Whether the streaming kernel takes this lane-path launch: one activation
// row, group 64, K of 2048 or 6144, plain or swiglu, no group-sum output, at
// most 16384 rows (the decode step's projections).
// Q3VL_GEMV_STREAM=0 in the environment keeps every launch on gemv_kernel.
static bool stream_takes(const GemvArgs &a) {
    static const bool enabled = [] {
        const char *v = getenv("Q3VL_GEMV_STREAM");
        return !(v && v[0] == '0');
    }();
    if (!enabled || a.M != 1 || a.gs != 64 || (a.K != 2048 && a.K != 6144)) return false;
    if (a.mode != GEMV_PLAIN && a.mode != GEMV_SWIGLU) return false;
    if (a.mode == GEMV_SWIGLU && (a.nseg != 2 || a.K != 2048)) return false;
    if (a.norm_w && a.K != 2048) return false;
    int rows = 0;
    for (int s = 0; s < a.nseg; ++s) {
        if (a.seg[s].G) return false;
        rows += a.seg[s].N;
    }
    // (the lm_head's 151936 rows stay on gemv_kernel's 8-row tiles: 56
    // against 64 us)
    return rows <= 16384;
}

static hipError_t launch_stream(const GemvArgs &a, int *grid_out, hipStream_t st) {
    const StreamCfg c = stream_cfg(a);
    if (a.K == 2048)
        return a.mode == GEMV_SWIGLU ? launch_stream_md<2048, MD_SWIGLU>(a, c, grid_out, st)
                                     : launch_stream_md<2048, MD_RUNTIME>(a, c, grid_out, st);
    return launch_stream_md<6144, MD_RUNTIME>(a, c, grid_out, st);
}

template <int GS>
static hipError_t launch_gemv_gs(const GemvArgs &a, bool lanes, int *grid_out, hipStream_t st) {
    if (lanes) {
        if (GS == 64 && stream_takes(a)) return launch_stream(a, grid_out, st);
        if (GS == 64 && a.K == 2048) {
            int dev = 0, cus = 0;
            hipError_t e = hipGetDevice(&dev);
            if (e == hipSuccess) e = device_cus(dev, &cus);
            if (e != hipSuccess) return e;
            switch (lane_rows_sub(a, cus)) {
                case 2: return launch_lanes<GS, 2, kSubGroups>(a, grid_out, st);
                case 4: return launch_lanes<GS, 4, kSubGroups>(a, grid_out, st);
                case 8: return launch_lanes<GS, 8, kSubGroups>(a, grid_out, st);
                default: break;  // one tile per block
            }
        }
        switch (lane_rows(a)) {
            case 2: return launch_lanes<GS, 2>(a, grid_out, st);
            case 4: return launch_lanes<GS, 4>(a, grid_out, st);
            default: return launch_lanes<GS, 8>(a, grid_out, st);
        }
    }
    if (a.M <= 1) return launch_gemv_t<GS, 1, false, GEMV_R>(a, grid_out, st);
    if (a.M <= 2) return launch_gemv_t<GS, 2, false, GEMV_R>(a, grid_out, st);
    if (a.M <= 4) return launch_gemv_t<GS, 4, false, GEMV_R>(a, grid_out, st);
    return launch_gemv_t<GS, 8, false, GEMV_R>(a, grid_out, st);
}

hipError_t launch_gemv(const GemvArgs &a, bool lanes, int *grid_out, hipStream_t st) {
    if (a.M < 1 || a.M > 8 || a.K % 16 != 0 || a.K / 16 > GEMV_MAX_THREADS)
        return hipErrorInvalidValue;
    if (a.norm_w && (a.M != 1 || !a.norm_s)) return hipErrorInvalidValue;
    switch (a.gs) {
        case 16: return launch_gemv_gs<16>(a, lanes, grid_out, st);
        case 32: return launch_gemv_gs<32>(a, lanes, grid_out, st);
        case 64: return launch_gemv_gs<64>(a, lanes, grid_out, st);
        case 128: return launch_gemv_gs<128>(a, lanes, grid_out, st);
        case 256: return launch_gemv_gs<256>(a, lanes, grid_out, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_argmax_final(const float *pv, const int32_t *pi, int nparts, int M,
                               int32_t *ids, hipStream_t st, int32_t *pos_inc) {
    // (the kernel clamps its loads to partial nparts - 1: at least one)
    if (nparts < 1 || nparts > 8192) return hipErrorInvalidValue;
    if (M < 1) return hipErrorInvalidValue;
    argmax_final_kernel<<<M, 256, 0, st>>>(pv, pi, nparts, M, ids, pos_inc);
    return hipGetLastError();
}

hipError_t launch_argmax_partials(const float *logits, int M, int V, float *pv, int32_t *pi,
                                  int nparts, hipStream_t st) {
    argmax_part_kernel<<<dim3(nparts, M), 256, 0, st>>>(logits, M, V, nparts, pv, pi);
    return hipGetLastError();
}

hipError_t launch_argmax_rows(const float *logits, int M, int V, float *pv, int32_t *pi,
                              int nparts, int32_t *ids, hipStream_t st) {
    hipError_t e = launch_argmax_partials(logits, M, V, pv, pi, nparts, st);
    if (e != hipSuccess) return e;
    return launch_argmax_final(pv, pi, nparts, M, ids, st);
}

// n 32-bit words set to zero, as a kernel: a call captured into a HIP graph
// then records a kernel node, not a memset node (memset nodes have given
// wrong results on replays after the first on this platform).
__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t *p, size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = 0u;
}

hipError_t launch_zero_words(void *p, size_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    const size_t blocks = (n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096;
    zero_words_kernel<<<(unsigned)blocks, 256, 0, st>>>(static_cast<uint32_t *>(p), n);
    return hipGetLastError();
}

hipError_t launch_swiglu(float *gate, const float *up, size_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    swiglu_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(gate, up, n);
    return hipGetLastError();
}

}  // namespace q3vl
