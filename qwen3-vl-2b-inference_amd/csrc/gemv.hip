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

#include "q3vl_device.hpp"
#include "q3vl_kernels.hpp"

namespace q3vl {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int GEMV_R = 8;          // weight rows per tile
constexpr int GEMV_MAX_THREADS = 512;  // => K <= 8192 on this path
constexpr int GEMV_MAX_GRID = 8192;    // the C ABI reserves this many argmax partials

// SwiGLU epilogue, layers/src/text_layer.cpp:428-433:
// silu = g / (1 + expf(-g)); h = silu * u. exp is evaluated in double and
// rounded once (a correctly rounded expf except for halfway-close cases);
// the division is correctly rounded as in the fp32 reference.
__device__ __forceinline__ float silu_mul(float gv, float uv) {
    const float e = (float)::exp(-(double)gv);
    const float den = 1.0f + e;
    const float sl = (float)((double)gv / (double)den);
    return sl * uv;
}

template <int GS, int MR, bool LANES>
__global__ __launch_bounds__(GEMV_MAX_THREADS) void gemv_kernel(GemvArgs a, int ntiles) {
    constexpr int T = GS / 16;
    constexpr int R = GEMV_R;
    extern __shared__ __align__(16) unsigned char smem[];

    const int K = a.K;
    const int Kg = K / GS;
    const int M = a.M;
    const int tid = threadIdx.x;
    const int nthr = blockDim.x;
    const int g = tid / T;
    const int tg = tid % T;

    // ---- LDS carve-up
    const int acc_words = LANES ? R * (8 * Kg + 8) : MR * R * (Kg + 1);
    const int stage_words = acc_words > K ? acc_words : K;
    int32_t *accb = reinterpret_cast<int32_t *>(smem);
    float *xs = reinterpret_cast<float *>(smem);  // phase 0 only (aliases accb)
    float *as_l = reinterpret_cast<float *>(smem) + stage_words;  // [M][Kg]
    float *sc_l = as_l + MR * Kg;                                   // [R][Kg]
    float *ybuf = sc_l + R * Kg;                                    // [MR][R]

    // ---- phase 0: quantize the activation rows (reference i8:135-177)
    uint32_t qp[MR][8];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
#pragma unroll
        for (int j = 0; j < 8; ++j) qp[m][j] = 0;
        if (m >= M) continue;  // uniform: every thread skips together
        const float4 *src = reinterpret_cast<const float4 *>(a.A + (size_t)m * K);
        for (int i = tid; i < K / 4; i += nthr) reinterpret_cast<float4 *>(xs)[i] = src[i];
        __syncthreads();
        // Every thread of a group recomputes the group's sum of squares from
        // LDS in the reference order: 16 FMA chains over the gs/16 steps,
        // then the fixed tree.
        float P[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) P[i] = 0.0f;
        const float *xg = xs + g * GS;
#pragma unroll
        for (int t = 0; t < T; ++t) {
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                const float4 v = reinterpret_cast<const float4 *>(xg + 16 * t)[i4];
                P[4 * i4 + 0] = fmaf(v.x, v.x, P[4 * i4 + 0]);
                P[4 * i4 + 1] = fmaf(v.y, v.y, P[4 * i4 + 1]);
                P[4 * i4 + 2] = fmaf(v.z, v.z, P[4 * i4 + 2]);
                P[4 * i4 + 3] = fmaf(v.w, v.w, P[4 * i4 + 3]);
            }
        }
        float V[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) V[i] = P[i] + P[i + 8];
        const float sumsq = tree8(V[0], V[1], V[2], V[3], V[4], V[5], V[6], V[7]);
        const float s = group_scale(sumsq, 1.0f / (float)GS);
        const float inv = rcp_rn(s);
        if (tg == 0) as_l[m * Kg + g] = s;
        const float *xc = xs + 16 * tid;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int32_t lo = quant_cvt(xc[2 * j] * inv);
            const int32_t hi = quant_cvt(xc[2 * j + 1] * inv);
            qp[m][j] = ((uint32_t)lo & 0xFFFFu) | ((uint32_t)hi << 16);
        }
        __syncthreads();
    }

    // Running argmax of activation row `tid` (threads tid < M), over the
    // block's tiles in ascending row order.
    float best = -FLT_MAX;
    int32_t bidx = -1;

    const int half = R / 2;
    for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        // ---- resolve the tile's rows: row r of the tile is row tn0 + r of
        // segment tseg (plain / argmax), or row tn0 + r % (R/2) of the gate
        // (r < R/2) or up segment (swiglu).
        const bool swg = a.mode == GEMV_SWIGLU;
        int tseg = 0, tn0;
        if (swg) {
            tn0 = tile * half;
        } else {
            int t0 = tile;
            while (tseg + 1 < a.nseg) {
                const int ts = (a.seg[tseg].N + R - 1) / R;
                if (t0 < ts) break;
                t0 -= ts;
                ++tseg;
            }
            tn0 = t0 * R;
        }
        const int tN = a.seg[tseg].N;
        auto row_seg = [&](int r) { return swg ? (r < half ? 0 : 1) : tseg; };
        auto row_n = [&](int r) { return swg ? tn0 + (r & (half - 1)) : tn0 + r; };
        auto row_ok = [&](int r) { return row_n(r) < tN; };
        bool valid[R];
        const int8_t *wrow[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            valid[r] = row_ok(r);
            wrow[r] = a.seg[row_seg(r)].W + (size_t)(valid[r] ? row_n(r) : 0) * K;
        }

        // ---- issue all weight loads of the tile
        u32x4 wv[R];
#pragma unroll
        for (int r = 0; r < R; ++r)
            wv[r] = valid[r] ? __builtin_nontemporal_load(
                                   reinterpret_cast<const u32x4 *>(wrow[r]) + tid)
                             : (u32x4){0u, 0u, 0u, 0u};

        // ---- scales of the tile's rows -> LDS
        for (int i = tid; i < R * Kg; i += nthr) {
            const int r = i / Kg, gg = i - r * Kg;
            float v = 0.0f;
            if (row_ok(r)) {
                const float ws = a.seg[row_seg(r)].S[(size_t)row_n(r) * Kg + gg];
                v = LANES ? as_l[gg] * ws : ws;  // i8:213 a_s * w_s (lanes)
            }
            sc_l[i] = v;
        }

        // ---- phase 1: exact integer lane / group sums
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (!valid[r]) continue;  // uniform across the block
            const uint32_t wd[4] = {wv[r].x, wv[r].y, wv[r].z, wv[r].w};
            uint32_t wp[8];
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                wp[2 * d] = lo2(wd[d]);
                wp[2 * d + 1] = hi2(wd[d]);
            }
            if constexpr (LANES) {
                int32_t p[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) p[j] = run_sum<T>(dot2(qp[0][j], wp[j], 0));
                if (tg == 0) {
                    int4 *dst = reinterpret_cast<int4 *>(accb + r * (8 * Kg + 8) + 8 * g);
                    dst[0] = make_int4(p[0] >> 8, p[1] >> 8, p[2] >> 8, p[3] >> 8);
                    dst[1] = make_int4(p[4] >> 8, p[5] >> 8, p[6] >> 8, p[7] >> 8);
                    int32_t *Gd = a.seg[row_seg(r)].G;
                    if (Gd) {
                        int32_t tot = 0;
#pragma unroll
                        for (int j = 0; j < 8; ++j) tot += p[j] >> 8;
                        Gd[(size_t)row_n(r) * Kg + g] = tot;
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
                    if (tg == 0) {
                        accb[(m * R + r) * (Kg + 1) + g] = acc;
                        int32_t *Gd = a.seg[row_seg(r)].G;
                        if (Gd) Gd[((size_t)m * tN + row_n(r)) * Kg + g] = acc;
                    }
                }
            }
        }
        __syncthreads();

        // ---- phase 2: fp32 group chains in the reference order
        float y = 0.0f;
        int ym = 0, yr = 0;
        bool yvalid = false;
        if constexpr (LANES) {
            if (tid < 8 * R) {
                const int r = tid >> 3, j = tid & 7;
                float c = 0.0f;
                if (row_ok(r)) {
                    const int32_t *Lr = accb + r * (8 * Kg + 8) + j;
                    const float *scr = sc_l + r * Kg;
                    for (int gg = 0; gg < Kg; ++gg)
                        c = fmaf((float)Lr[8 * gg], scr[gg], c);  // i8:213-216
                }
                // add_reduce_mm_256 over the row's 8 lanes (i8:219-222).
                c = c + __shfl_xor(c, 4, 8);
                c = c + __shfl_xor(c, 1, 8);
                c = c + __shfl_xor(c, 2, 8);
                y = c;
                ym = 0;
                yr = r;
                yvalid = (j == 0) && row_ok(r);
            }
        } else {
            if (tid < M * R) {
                const int m = tid / R, r = tid - (tid / R) * R;
                float acc = 0.0f;
                if (row_ok(r)) {
                    const int32_t *Gr = accb + (m * R + r) * (Kg + 1);
                    const float *asr = as_l + m * Kg;
                    const float *wsr = sc_l + r * Kg;
                    for (int gg = 0; gg < Kg; ++gg) {
                        const float ga = (float)Gr[gg] * asr[gg];
                        acc = fmaf(ga, wsr[gg], acc);  // i8:613-617 (contracted)
                    }
                }
                y = acc;
                ym = m;
                yr = r;
                yvalid = row_ok(r);
            }
        }

        // ---- epilogues
        if (a.mode == GEMV_PLAIN) {
            if (yvalid) a.seg[row_seg(yr)].Y[(size_t)ym * tN + row_n(yr)] = y;
        } else {
            if (yvalid) ybuf[ym * R + yr] = y;
            __syncthreads();
            if (a.mode == GEMV_SWIGLU) {
                if (tid < M * half) {
                    const int m = tid / half, r = tid - (tid / half) * half;
                    if (row_ok(r))
                        a.seg[0].Y[(size_t)m * tN + row_n(r)] =
                            silu_mul(ybuf[m * R + r], ybuf[m * R + r + half]);
                }
            } else {  // GEMV_ARGMAX
                if (tid < M) {
                    const int m = tid;
                    for (int r = 0; r < R; ++r) {
                        if (!row_ok(r)) break;
                        const float v = ybuf[m * R + r];
                        if (a.seg[0].Y) a.seg[0].Y[(size_t)m * tN + row_n(r)] = v;
                        // greedy_decode (tokenizer/src/utils.cpp:34-44): strict >
                        if (v > best) {
                            best = v;
                            bidx = row_n(r);
                        }
                    }
                }
            }
        }
        __syncthreads();
    }

    if (a.mode == GEMV_ARGMAX && tid < M) {
        a.part_val[(size_t)blockIdx.x * M + tid] = best;
        a.part_idx[(size_t)blockIdx.x * M + tid] = bidx;
    }
}

// ----------------------------------------------------------------- argmax
// Combine rule equivalent to the sequential strict-> scan: the larger value
// wins, equal values keep the lower index, candidates with idx<0 are empty.
__device__ __forceinline__ void am_combine(float &bv, int32_t &bi, float v, int32_t i) {
    if (i < 0) return;
    if (bi < 0 || v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
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

__global__ __launch_bounds__(256) void argmax_final_kernel(const float *pv, const int32_t *pi,
                                                           int nparts, int M, int32_t *ids) {
    for (int m = 0; m < M; ++m) {
        float bv = -FLT_MAX;
        int32_t bi = -1;
        for (int p = threadIdx.x; p < nparts; p += blockDim.x)
            am_combine(bv, bi, pv[(size_t)p * M + m], pi[(size_t)p * M + m]);
        am_block_reduce(bv, bi);
        if (threadIdx.x == 0) ids[m] = bi < 0 ? 0 : bi;
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
template <int GS, int MR, bool LANES>
static hipError_t launch_gemv_t(const GemvArgs &a, int *grid_out, hipStream_t st) {
    constexpr int R = GEMV_R;
    const int K = a.K, Kg = K / GS;
    const int nthr = K / 16;
    const int acc_words = LANES ? R * (8 * Kg + 8) : MR * R * (Kg + 1);
    const int stage_words = acc_words > K ? acc_words : K;
    const size_t lds = (size_t)(stage_words + MR * Kg + R * Kg + MR * R) * 4;

    int ntiles = 0;
    if (a.mode == GEMV_SWIGLU) {
        ntiles = (a.seg[0].N + R / 2 - 1) / (R / 2);
    } else {
        for (int s = 0; s < a.nseg; ++s) ntiles += (a.seg[s].N + R - 1) / R;
    }
    int dev = 0, cus = 0, occ = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return e;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, gemv_kernel<GS, MR, LANES>, nthr, lds);
    if (e != hipSuccess) return e;
    if (occ < 1) occ = 1;
    int grid = cus * occ;
    if (grid > GEMV_MAX_GRID) grid = GEMV_MAX_GRID;  // argmax partials reserved per launch
    if (grid > ntiles) grid = ntiles;
    if (grid < 1) grid = 1;
    if (grid_out) *grid_out = grid;
    gemv_kernel<GS, MR, LANES><<<grid, nthr, lds, st>>>(a, ntiles);
    return hipGetLastError();
}

template <int GS>
static hipError_t launch_gemv_gs(const GemvArgs &a, bool lanes, int *grid_out, hipStream_t st) {
    if (lanes) return launch_gemv_t<GS, 1, true>(a, grid_out, st);
    if (a.M <= 1) return launch_gemv_t<GS, 1, false>(a, grid_out, st);
    if (a.M <= 2) return launch_gemv_t<GS, 2, false>(a, grid_out, st);
    if (a.M <= 4) return launch_gemv_t<GS, 4, false>(a, grid_out, st);
    return launch_gemv_t<GS, 8, false>(a, grid_out, st);
}

hipError_t launch_gemv(const GemvArgs &a, bool lanes, int *grid_out, hipStream_t st) {
    if (a.M < 1 || a.M > 8 || a.K % 16 != 0 || a.K / 16 > GEMV_MAX_THREADS)
        return hipErrorInvalidValue;
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
                               int32_t *ids, hipStream_t st) {
    argmax_final_kernel<<<1, 256, 0, st>>>(pv, pi, nparts, M, ids);
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

hipError_t launch_swiglu(float *gate, const float *up, size_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    swiglu_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(gate, up, n);
    return hipGetLastError();
}

}  // namespace q3vl
