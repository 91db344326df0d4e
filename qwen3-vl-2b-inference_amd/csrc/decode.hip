// decode.hip -- support kernels of the text decode step that calls the int8
// path (model/src/forward.cpp:458-720), gfx950.
//
// Every floating-point step follows the reference's order, including the
// orders its compiler picks for `omp simd` reductions on 8-wide AVX2: the
// RMS sums of squares and the scores of the last partial block of 8
// positions use 8 FMA lane chains folded left to right, the softmax sums 8
// float lanes then adds them in double, and the value-weighted sum is one
// FMA chain over positions per output element. The decode step is therefore
// bit-exact with the CPU oracle in its fp16-cache mode.
#include <float.h>

#include "q3vl_device.hpp"
#include "q3vl_kernels.hpp"

namespace q3vl {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ helpers
// layers/include/simd_utils.hpp:7-47 exp256_ps, one lane (2^n is -inf for
// n = -128, as in the reference).
__device__ __forceinline__ float exp256(float x) {
    x = fminf(x, 88.3762626647949f);
    x = fmaxf(x, -88.3762626647949f);
    const float ln2 = 0.69314718056f, inv_ln2 = 1.44269504089f;
    const float fx = floorf(x * inv_ln2);
    const int32_t n = (int32_t)fx;
    const float g = fmaf(-fx, ln2, x);
    float y = fmaf(g, 1.0f, 1.0f);
    const float g2 = g * g;
    y = fmaf(g2, 0.5f, y);
    const float g3 = g2 * g;
    y = fmaf(g3, 1.0f / 6.0f, y);
    const float g4 = g3 * g;
    y = fmaf(g4, 1.0f / 24.0f, y);
    return y * __uint_as_float((uint32_t)(n + 127) << 23);
}

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
// fp32 -> fp16 bits, round to nearest even, computed on the integer image.
// A plain (_Float16) conversion lets the compiler fuse it with the fmaf that
// produced the value (v_fma_mixlo_f16 rounds the exact result once, straight
// to fp16), which differs from the reference's fp32 result rounded to fp16
// whenever that result lies exactly halfway between two fp16 values.
__device__ __forceinline__ uint16_t f2h(float f) {
    const uint32_t x = __float_as_uint(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);  // rounds past 65504
    if (ax < 0x33000000u) return (uint16_t)sign;                // at most 2^-25: zero
    uint32_t r, rem, half;
    if (ax < 0x38800000u) {  // fp16 subnormal: keep the bits above 2^-24
        const uint32_t shift = 126u - (ax >> 23);  // 14..24
        const uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        r = m >> shift;
        rem = m & ((1u << shift) - 1u);
        half = 1u << (shift - 1u);
    } else {                 // normal: rebias the exponent, drop 13 mantissa bits
        r = (ax >> 13) - (112u << 10);
        rem = ax & 0x1FFFu;
        half = 0x1000u;
    }
    r += (rem > half || (rem == half && (r & 1u))) ? 1u : 0u;
    return (uint16_t)(sign | r);
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Left-to-right fold of the 8 lane accumulators held by lanes 0..7:
// ((c0 + c1) + c2) + ... + c7; wave-uniform result.
__device__ __forceinline__ float fold8_lanes(float c) {
    float s = readlane_f(c, 0);
#pragma unroll
    for (int l = 1; l < 8; ++l) s = s + readlane_f(c, l);
    return s;
}

// Sum of squares of a 128-vector held by one wave as (lo = x[lane],
// hi = x[lane + 64]) in the reference's order (text_layer.cpp:247-250 as
// compiled): chain c = lane & 7 takes x[c], x[c+8], ..., x[c+120] with one
// FMA each -- lo of lanes c, c+8, ..., c+56, then hi of the same lanes --
// and the 8 chains are folded left to right.
__device__ __forceinline__ float wave_sumsq128(float lo, float hi) {
    const int c = __lane_id() & 7;
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const float v = __shfl(lo, c + 8 * k);
        acc = fmaf(v, v, acc);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const float v = __shfl(hi, c + 8 * k);
        acc = fmaf(v, v, acc);
    }
    return fold8_lanes(acc);
}

// layers/src/text_layer.cpp:240-270 (int8 group weight, in place) on one
// head of 128 held by a wave, then RoPE (text_layer.cpp:712-760) with the
// pair (x[i], x[i+64]) in one lane.
__device__ __forceinline__ void norm_rope128(float &lo, float &hi, const int8_t *w, const float *ws,
                                             int gs, float eps, float c, float s, int lane) {
    const float ss = wave_sumsq128(lo, hi);
    const float inv = rcp_rn(sqrt_rn(ss * (1.0f / 128.0f) + eps));  // 1.0f / sqrtf(...)
    lo = (float)w[lane] * ((ws[lane / gs] * inv) * lo);
    hi = (float)w[lane + 64] * ((ws[(lane + 64) / gs] * inv) * hi);
    const float a = lo, b = hi;
    lo = fmaf(a, c, -(b * s));
    hi = fmaf(a, s, b * c);
}

// ----------------------------------------------------------------- embedding
// layers/src/text_layer.cpp:3-49, int8 group-quantized table.
__global__ __launch_bounds__(256) void embed_kernel(const int8_t *w, const float *s,
                                                    const int32_t *token, float *x, int H,
                                                    int gs) {
    const size_t base = (size_t)(*token) * H;
    for (int i = threadIdx.x + blockIdx.x * blockDim.x; i < H; i += blockDim.x * gridDim.x)
        x[i] = (float)w[base + i] * s[(base + i) / gs];
}

// --------------------------------------------------------------- attention
// A: per (kv head, chunk of ATT_CH positions), one wave per query head of the
// group. The waves normalize + rotate their query heads (q RMSNorm + RoPE,
// forward.cpp:531-545); the chunk holding `pos` also normalizes + rotates the
// new key and stores it and the new value as fp16 at pos (forward.cpp:
// 548-562). Scores follow text_layer.cpp:598-620 exactly: 8 FMA lane chains
// over the head dimension, the fixed tree (the left-to-right fold for the
// positions of the last partial block of 8), times 1/sqrt(hd).
constexpr int ATT_CH = 64;
constexpr int ATT_HD = 128;
constexpr int ATT_KSTR = ATT_HD + 8;  // halves per LDS key row (272 B: bank-spread)

__global__ __launch_bounds__(256) void attn_scores_kernel(AttnArgs a) {
    __shared__ float qsh[4][ATT_HD];
    __shared__ uint16_t ksh[ATT_CH * ATT_KSTR];
    __shared__ uint16_t knew[ATT_HD];
    const int kvh = blockIdx.x, ch = blockIdx.y;
    const int pos = *a.pos;
    const int n = pos + 1;
    const int t0 = ch * ATT_CH;
    if (t0 >= n) return;  // uniform: chunk past the context
    const int kvm = a.heads / a.kv_heads;
    const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const float c = a.rope_cos[(size_t)pos * (ATT_HD / 2) + lane];
    const float s = a.rope_sin[(size_t)pos * (ATT_HD / 2) + lane];
    const size_t lay = (size_t)a.layer * a.kv_heads * a.max_seq * ATT_HD;
    uint16_t *kc = a.k_cache + lay + (size_t)kvh * a.max_seq * ATT_HD;
    uint16_t *vc = a.v_cache + lay + (size_t)kvh * a.max_seq * ATT_HD;
    const bool own_pos = pos >= t0 && pos < t0 + ATT_CH;

    if (wid < kvm) {
        const int h = kvh * kvm + wid;
        float lo = a.q[h * ATT_HD + lane], hi = a.q[h * ATT_HD + 64 + lane];
        norm_rope128(lo, hi, a.qnorm_w, a.qnorm_s, a.gs, a.eps, c, s, lane);
        qsh[wid][lane] = lo;
        qsh[wid][lane + 64] = hi;
    } else if (wid == kvm && own_pos) {
        float lo = a.k[kvh * ATT_HD + lane], hi = a.k[kvh * ATT_HD + 64 + lane];
        norm_rope128(lo, hi, a.knorm_w, a.knorm_s, a.gs, a.eps, c, s, lane);
        const uint16_t l16 = f2h(lo), h16 = f2h(hi);
        kc[(size_t)pos * ATT_HD + lane] = l16;
        kc[(size_t)pos * ATT_HD + 64 + lane] = h16;
        knew[lane] = l16;
        knew[lane + 64] = h16;
        vc[(size_t)pos * ATT_HD + lane] = f2h(a.v[kvh * ATT_HD + lane]);
        vc[(size_t)pos * ATT_HD + 64 + lane] = f2h(a.v[kvh * ATT_HD + 64 + lane]);
    }
    // key tile of the chunk -> LDS (rows at or past pos come from knew)
    const int rows = min(ATT_CH, n - t0);
    for (int i = threadIdx.x; i < ATT_CH * (ATT_HD / 8); i += blockDim.x) {
        const int r = i / (ATT_HD / 8), c8 = i % (ATT_HD / 8);
        u32x4 v = (u32x4){0u, 0u, 0u, 0u};
        if (r < rows && t0 + r != pos)
            v = *reinterpret_cast<const u32x4 *>(kc + (size_t)(t0 + r) * ATT_HD + c8 * 8);
        *reinterpret_cast<u32x4 *>(ksh + r * ATT_KSTR + c8 * 8) = v;
    }
    __syncthreads();
    if (own_pos && threadIdx.x < ATT_HD) ksh[(pos - t0) * ATT_KSTR + threadIdx.x] = knew[threadIdx.x];
    __syncthreads();
    if (wid >= kvm) return;
    const int h = kvh * kvm + wid;
    const int t = t0 + lane;
    float score = -INFINITY;
    if (lane < rows) {
        float cc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        const uint16_t *kr = ksh + lane * ATT_KSTR;
#pragma unroll
        for (int i = 0; i < ATT_HD; i += 8) {
            const u32x4 kk = *reinterpret_cast<const u32x4 *>(kr + i);
            const uint32_t kw[4] = {kk.x, kk.y, kk.z, kk.w};
#pragma unroll
            for (int l = 0; l < 8; ++l) {
                const uint16_t hb = (uint16_t)(kw[l >> 1] >> (16 * (l & 1)));
                cc[l] = fmaf(qsh[wid][i + l], h2f(hb), cc[l]);
            }
        }
        float dot;
        if (t >= (pos & ~7)) {  // text_layer.cpp:626-633: lanes folded left to right
            dot = cc[0];
#pragma unroll
            for (int l = 1; l < 8; ++l) dot = dot + cc[l];
        } else {                // text_layer.cpp:598-620: the fixed tree
            dot = tree8(cc[0], cc[1], cc[2], cc[3], cc[4], cc[5], cc[6], cc[7]);
        }
        score = dot * a.inv_sqrt_d;
        a.scores[(size_t)h * a.max_seq + t] = score;
    }
    float m = score;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if (lane == 0) a.cmax[h * a.max_chunks + ch] = m;
}

// B: softmax (text_layer.cpp:436-535) and the value-weighted sum
// (text_layer.cpp:655-710) in the reference's order. Block (kv head kvh,
// slice db) serves the kvm query heads of kvh and the PV_D output dims
// [db*PV_D, db*PV_D + PV_D). Per head:
//   M = max of the scores (exact: the scores kernel's chunk maxima),
//   e_t = exp256(s_t - M) (0 for s_t = -inf),
//   sum = double(l_0) + ... + double(l_7) + e_nb + ... + e_pos (in double),
//     l_j = sequential fp32 sum of e_t over t = j (mod 8), t < nb = n/8*8,
//   p_t = e_t * (float)(1/sum)   (all zero if M or sum is not finite/positive),
//   out[d] = fma chain over t = 0..pos of p_t * v_t[d].
// The chain is inherently sequential (one dependent FMA per position), so
// everything else is arranged to keep it to one v_fmac_f32 per step: every
// global load (the first V chunk, the chunk maxima, up to PV_SREG*PV_THREADS
// scores per head) is issued at entry; V is widened to fp32 into LDS,
// transposed ([d][t]); p is formed in LDS before the chains start; the chains
// read 32 positions ahead. e also lives lane-major (row j holds e_j, e_{j+8},
// ...) so the 8 summing lanes read contiguous 16-byte words.
constexpr int PV_D = 16;
constexpr int PV_TC = 1024;
constexpr int PV_THREADS = 256;
constexpr int PV_RS = PV_TC + 4;                    // floats per LDS row of vt
constexpr int PV_ITEMS = PV_TC * (PV_D / 8) / PV_THREADS;  // (position, 8-dim segment) items
constexpr int PV_SREG = 8;                          // scores held in registers per head

// Lane-major e rows hold max_seq/8 terms rounded up to a multiple of 32 (the
// summing batch), plus 4 floats of padding against bank conflicts.
__host__ __device__ __forceinline__ int pv_et_stride(int max_seq) {
    return (max_seq / 8 + 31) / 32 * 32 + 4;
}

__global__ __launch_bounds__(PV_THREADS) void attn_softmax_pv_kernel(AttnArgs a) {
    extern __shared__ __align__(16) float smem[];
    const int kvm = a.heads / a.kv_heads;
    const int S = a.max_seq, ets = pv_et_stride(S);
    float *vt = smem;                       // [PV_D][PV_RS] fp32
    float *e = smem + PV_D * PV_RS;         // [kvm][S]: e_t, then p_t
    float *et = e + kvm * S;                // [kvm][8][ets]
    __shared__ float hmax[4], hinv[4];
    const int kvh = blockIdx.x, db = blockIdx.y;
    const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63;
    const int n = *a.pos + 1;
    const int nb = n & ~7;
    const uint16_t *vc = a.v_cache + ((size_t)a.layer * a.kv_heads + kvh) * S * ATT_HD + db * PV_D;

    // V chunk loads: item -> (8-dim segment sg, position t), one 16-byte
    // load each, clamped into the context.
    u32x4 vr[PV_ITEMS];
    auto load_chunk = [&](int t0) {
#pragma unroll
        for (int it = 0; it < PV_ITEMS; ++it) {
            const int item = it * PV_THREADS + tid;
            const int sg = item / PV_TC, t = t0 + item % PV_TC;
            vr[it] = *reinterpret_cast<const u32x4 *>(vc + (size_t)min(t, n - 1) * ATT_HD + sg * 8);
        }
    };
    auto store_chunk = [&]() {
#pragma unroll
        for (int it = 0; it < PV_ITEMS; ++it) {
            const int item = it * PV_THREADS + tid;
            const int sg = item / PV_TC, t = item % PV_TC;
            const uint32_t w[4] = {vr[it].x, vr[it].y, vr[it].z, vr[it].w};
#pragma unroll
            for (int i = 0; i < 8; ++i)
                vt[(sg * 8 + i) * PV_RS + t] = h2f((uint16_t)(w[i >> 1] >> (16 * (i & 1))));
        }
    };
    load_chunk(0);

    // scores of this thread's positions t = tid + PV_THREADS*k, k < PV_SREG
    float sreg[3][PV_SREG];
#pragma unroll
    for (int hh = 0; hh < 3; ++hh) {
        if (hh < kvm) {
            const float *sc = a.scores + (size_t)(kvh * kvm + hh) * S;
#pragma unroll
            for (int k = 0; k < PV_SREG; ++k) sreg[hh][k] = sc[min(tid + PV_THREADS * k, n - 1)];
        }
    }
    // maxima from the chunk maxima, one wave per head
    const int nch = (n + ATT_CH - 1) / ATT_CH;
    if (wid < kvm) {
        const int h = kvh * kvm + wid;
        float m = -INFINITY;
        for (int c = lane; c < nch; c += 64) m = fmaxf(m, a.cmax[h * a.max_chunks + c]);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        if (lane == 0) hmax[wid] = m;
    }
    lds_barrier();
    // e_t (text_layer.cpp:486-493, 501-509), stored both ways
#pragma unroll
    for (int hh = 0; hh < 3; ++hh) {
        if (hh < kvm) {
            const float M = hmax[hh];
            const bool fin = __builtin_isfinite(M);
            float *eh = e + hh * S, *eth = et + hh * 8 * ets;
            auto put = [&](int t, float v) {
                const float ev = (fin && v > -INFINITY) ? exp256(v - M) : 0.0f;
                eh[t] = ev;
                if (t < nb) eth[(t & 7) * ets + (t >> 3)] = ev;
            };
            // zeros after the lane sums' last term, up to a whole batch of 32
            // per lane: adding +0 to a sum of non-negative terms is exact
            const int zend = (nb + 255) & ~255;
            for (int t = nb + tid; t < zend; t += PV_THREADS) eth[(t & 7) * ets + (t >> 3)] = 0.0f;
#pragma unroll
            for (int k = 0; k < PV_SREG; ++k) {
                const int t = tid + PV_THREADS * k;
                if (t < n) put(t, sreg[hh][k]);
            }
            const float *sc = a.scores + (size_t)(kvh * kvm + hh) * S;
            for (int t = tid + PV_THREADS * PV_SREG; t < n; t += PV_THREADS) put(t, sc[t]);
        }
    }
    store_chunk();  // V chunk 0 (its loads were issued at entry)
    lds_barrier();
    // sums and the fp32 inverse, lanes 0..7 of one wave per head
    if (wid < kvm) {
        const float *row = et + wid * 8 * ets + (lane & 7) * ets;
        const int cnt = ((nb >> 3) + 31) & ~31;  // terms per lane, zero-padded
        float ls = 0.0f;
        if (lane < 8 && cnt > 0) {
            float4 A[8], B[8];
            auto ld = [&](float4 *D, int i) {
#pragma unroll
                for (int u = 0; u < 8; ++u) D[u] = *reinterpret_cast<const float4 *>(row + i + 4 * u);
            };
            auto add = [&](const float4 *D) {
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    ls = ls + D[u].x;
                    ls = ls + D[u].y;
                    ls = ls + D[u].z;
                    ls = ls + D[u].w;
                }
            };
            ld(A, 0);
            int i = 0;
            for (; i + 64 <= cnt; i += 64) {
                ld(B, i + 32);
                __builtin_amdgcn_sched_barrier(0);
                add(A);
                __builtin_amdgcn_sched_barrier(0);
                ld(A, min(i + 64, cnt - 32));
                __builtin_amdgcn_sched_barrier(0);
                add(B);
                __builtin_amdgcn_sched_barrier(0);
            }
            if (i < cnt) add(A);  // one batch of 32 left
        }
        double sum = 0.0;
#pragma unroll
        for (int l = 0; l < 8; ++l) sum += (double)readlane_f(ls, l);
        const float *eh = e + wid * S;
        for (int t = nb; t < n; ++t) sum += (double)eh[t];
        const bool ok = __builtin_isfinite(hmax[wid]) && sum > 0.0 && __builtin_isfinite(sum);
        const float inv = ok ? (float)(1.0 / sum) : 0.0f;
        if (lane == 0) hinv[wid] = inv;
    }
    lds_barrier();
    // p_t = e_t * inv, in place (four positions per thread per pass, reads first)
    for (int hh = 0; hh < kvm; ++hh) {
        const float inv = hinv[hh];
        float *eh = e + hh * S;
        for (int t0 = 0; t0 < n; t0 += 4 * PV_THREADS) {
            float v[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) v[k] = eh[min(t0 + tid + k * PV_THREADS, n - 1)];
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (t0 + tid + k * PV_THREADS < n) eh[t0 + tid + k * PV_THREADS] = v[k] * inv;
        }
    }

    // value-weighted sums: lane (ch_h, ch_d) of wave 0 runs one chain
    const int ch_d = tid % PV_D, ch_h = tid / PV_D;
    const bool chain = ch_h < kvm;
    float acc = 0.0f;
    for (int t0 = 0; t0 < n; t0 += PV_TC) {
        if (t0 > 0) {
            lds_barrier();  // previous chains done with vt
            store_chunk();
        }
        lds_barrier();      // vt and p ready
        if (t0 + PV_TC < n) load_chunk(t0 + PV_TC);
        if (chain) {
            const float *ph = e + ch_h * S + t0;
            const float *vrow = vt + ch_d * PV_RS;
            const int len = min(PV_TC, n - t0);
            int t = 0;
            if (len >= 32) {
                // batches of 32 positions in two register sets used in turn:
                // the next batch's LDS reads are issued before the current
                // batch's FMAs (all reads < len), with no register copies
                float4 Av[8], Ap[8], Bv[8], Bp[8];
                auto ld = [&](float4 *V, float4 *P, int i) {
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        V[u] = *reinterpret_cast<const float4 *>(vrow + i + 4 * u);
                        P[u] = *reinterpret_cast<const float4 *>(ph + i + 4 * u);
                    }
                };
                auto fma32 = [&](const float4 *V, const float4 *P) {
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        acc = fmaf(P[u].x, V[u].x, acc);
                        acc = fmaf(P[u].y, V[u].y, acc);
                        acc = fmaf(P[u].z, V[u].z, acc);
                        acc = fmaf(P[u].w, V[u].w, acc);
                    }
                };
                ld(Av, Ap, 0);
                for (; t + 64 <= len; t += 64) {
                    ld(Bv, Bp, t + 32);
                    __builtin_amdgcn_sched_barrier(0);
                    fma32(Av, Ap);
                    __builtin_amdgcn_sched_barrier(0);
                    ld(Av, Ap, min(t + 64, (len - 32) & ~3));
                    __builtin_amdgcn_sched_barrier(0);
                    fma32(Bv, Bp);
                    __builtin_amdgcn_sched_barrier(0);
                }
                if (t + 32 <= len) {  // A holds positions t .. t+31
                    fma32(Av, Ap);
                    t += 32;
                }
            }
            for (; t < len; ++t) acc = fmaf(ph[t], vrow[t], acc);
        }
    }
    if (chain) a.out[(kvh * kvm + ch_h) * ATT_HD + db * PV_D + ch_d] = acc;
}

// ------------------------------------------------------------------ launch
hipError_t launch_embed(const int8_t *w, const float *s, const int32_t *token, float *x, int H,
                        int gs, hipStream_t st) {
    embed_kernel<<<(H + 255) / 256, 256, 0, st>>>(w, s, token, x, H, gs);
    return hipGetLastError();
}

size_t attention_lds_bytes(int heads, int kv_heads, int max_seq) {
    const size_t kvm = (size_t)(heads / kv_heads);
    return (size_t)PV_D * PV_RS * 4 + kvm * max_seq * 4 + kvm * 8 * (size_t)pv_et_stride(max_seq) * 4;
}

hipError_t launch_attention(const AttnArgs &a, hipStream_t st) {
    const int kvm = a.heads / a.kv_heads;
    if (a.head_dim != ATT_HD || a.heads % a.kv_heads != 0 || kvm < 1 || kvm > 3 ||
        a.max_seq % 8 != 0)
        return hipErrorInvalidValue;
    const size_t lds = attention_lds_bytes(a.heads, a.kv_heads, a.max_seq);
    if (lds > kAttnMaxLds) return hipErrorInvalidValue;
    attn_scores_kernel<<<dim3(a.kv_heads, a.max_chunks), 64 * (kvm + 1), 0, st>>>(a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    static int lds_set = 0;  // raise the dynamic LDS limit once per process
    if (!lds_set) {
        e = hipFuncSetAttribute(reinterpret_cast<const void *>(&attn_softmax_pv_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)kAttnMaxLds);
        if (e != hipSuccess) return e;
        lds_set = 1;
    }
    attn_softmax_pv_kernel<<<dim3(a.kv_heads, ATT_HD / PV_D), PV_THREADS, lds, st>>>(a);
    return hipGetLastError();
}

}  // namespace q3vl
