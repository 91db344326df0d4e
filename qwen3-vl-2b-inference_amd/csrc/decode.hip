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

// ----------------------------------------------------------------- RMS norm
// One block of 256 threads per row of n <= RMS_MAX (n % 8 == 0, n % gs == 0).
// rms_norm (text_layer.cpp:110-147) and rms_norm_inplace (text_layer.cpp:
// 234-270) with int8 group weights: ss in the 8-lane order, inv = 1 /
// sqrt(ss/n + eps) rounded to fp32 -- both functions give the same value:
// sqrtf of the fp32 argument, then an fp32 reciprocal or a double one
// rounded to fp32, which agree -- and out = w * ((s_g * inv) * x).
// Thread i owns x[8i .. 8i+7] (one item; more items when n > 2048) and
// writes them chain-major to LDS, xs[l][j] = x[l + 8j], so chain lane l
// reads its terms four at a time.
constexpr int RMS_MAX = 8192;
constexpr int RMS_RS = RMS_MAX / 8 + 4;  // floats per chain row (16-byte padded)

__global__ __launch_bounds__(256) void rmsnorm_i8_kernel(const float *x, const int8_t *w,
                                                         const float *ws, float *out, int n,
                                                         int gs, float eps) {
    __shared__ __align__(16) float xs[8 * RMS_RS];
    __shared__ float s_inv;
    const int items = n >> 3;
    for (int it = threadIdx.x; it < items; it += 256) {
        const float4 a = reinterpret_cast<const float4 *>(x)[2 * it];
        const float4 b = reinterpret_cast<const float4 *>(x)[2 * it + 1];
        xs[0 * RMS_RS + it] = a.x;
        xs[1 * RMS_RS + it] = a.y;
        xs[2 * RMS_RS + it] = a.z;
        xs[3 * RMS_RS + it] = a.w;
        xs[4 * RMS_RS + it] = b.x;
        xs[5 * RMS_RS + it] = b.y;
        xs[6 * RMS_RS + it] = b.z;
        xs[7 * RMS_RS + it] = b.w;
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        float acc = 0.0f;
        if (threadIdx.x < 8) {
            const float *row = xs + threadIdx.x * RMS_RS;
            int j = 0;
            for (; j + 32 <= items; j += 32) {
                float4 v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) v[u] = *reinterpret_cast<const float4 *>(row + j + 4 * u);
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    acc = fmaf(v[u].x, v[u].x, acc);
                    acc = fmaf(v[u].y, v[u].y, acc);
                    acc = fmaf(v[u].z, v[u].z, acc);
                    acc = fmaf(v[u].w, v[u].w, acc);
                }
            }
            for (; j < items; ++j) acc = fmaf(row[j], row[j], acc);
        }
        const float ss = fold8_lanes(acc);
        if (threadIdx.x == 0) s_inv = rcp_rn(sqrt_rn(ss * rcp_rn((float)n) + eps));
    }
    __syncthreads();
    const float inv = s_inv;
    for (int it = threadIdx.x; it < items; it += 256) {
        float v[8];
#pragma unroll
        for (int l = 0; l < 8; ++l) v[l] = xs[l * RMS_RS + it];
        const int j0 = 8 * it;
        const uint2 wq = *reinterpret_cast<const uint2 *>(w + j0);
        float o[8];
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            const int8_t wb = (int8_t)(((l < 4 ? wq.x : wq.y) >> (8 * (l & 3))) & 0xFF);
            o[l] = (float)wb * ((ws[(j0 + l) / gs] * inv) * v[l]);
        }
        reinterpret_cast<float4 *>(out)[2 * it] = make_float4(o[0], o[1], o[2], o[3]);
        reinterpret_cast<float4 *>(out)[2 * it + 1] = make_float4(o[4], o[5], o[6], o[7]);
    }
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
// p lives in LDS; V passes through LDS in chunks of PV_TC positions stored
// transposed ([d][t], two positions per dword) so a lane reads 8 positions
// of its dim with one 16-byte load; the chunk after the current one is
// already in flight while the chains run.
constexpr int PV_D = 32;
constexpr int PV_TC = 1024;
constexpr int PV_THREADS = 256;
constexpr int PV_RS = PV_TC / 2 + 4;                 // dwords per LDS row of vt
constexpr int PV_ITEMS = (PV_TC / 2) * (PV_D / 8) / PV_THREADS;  // position pairs x 8-dim segments

__global__ __launch_bounds__(PV_THREADS) void attn_softmax_pv_kernel(AttnArgs a) {
    extern __shared__ __align__(16) float smem[];
    uint32_t *vt = reinterpret_cast<uint32_t *>(smem);  // [PV_D][PV_RS]
    float *p = smem + PV_D * PV_RS;                     // [kvm][max_seq]
    __shared__ float hinfo[4], hinv[4];  // per head: M, 1/sum
    const int kvh = blockIdx.x, db = blockIdx.y;
    const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63;
    const int kvm = a.heads / a.kv_heads;
    const int n = *a.pos + 1;
    const int nb = n & ~7;
    const uint16_t *vc = a.v_cache + ((size_t)a.layer * a.kv_heads + kvh) * a.max_seq * ATT_HD +
                         db * PV_D;

    // V chunk loads: item i -> segment (8 dims) sg, position pair pp; two
    // 16-byte rows (t = 2pp, 2pp+1) per item, zero past the context.
    u32x4 r0[PV_ITEMS], r1[PV_ITEMS];
    auto load_chunk = [&](int t0) {
#pragma unroll
        for (int it = 0; it < PV_ITEMS; ++it) {
            const int item = it * PV_THREADS + tid;
            const int sg = item / (PV_TC / 2), pp = item % (PV_TC / 2);
            const int t = t0 + 2 * pp;
            const int ta = min(t, n - 1), tb = min(t + 1, n - 1);
            r0[it] = *reinterpret_cast<const u32x4 *>(vc + (size_t)ta * ATT_HD + sg * 8);
            r1[it] = *reinterpret_cast<const u32x4 *>(vc + (size_t)tb * ATT_HD + sg * 8);
        }
    };
    auto store_chunk = [&]() {
#pragma unroll
        for (int it = 0; it < PV_ITEMS; ++it) {
            const int item = it * PV_THREADS + tid;
            const int sg = item / (PV_TC / 2), pp = item % (PV_TC / 2);
            const uint32_t w0[4] = {r0[it].x, r0[it].y, r0[it].z, r0[it].w};
            const uint32_t w1[4] = {r1[it].x, r1[it].y, r1[it].z, r1[it].w};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t h0 = (w0[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
                const uint32_t h1 = (w1[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
                vt[(sg * 8 + i) * PV_RS + pp] = h0 | (h1 << 16);
            }
        }
    };
    load_chunk(0);

    // maxima from the chunk maxima
    const int nch = (n + ATT_CH - 1) / ATT_CH;
    if (wid < kvm) {
        const int h = kvh * kvm + wid;
        float m = -INFINITY;
        for (int c = lane; c < nch; c += 64) m = fmaxf(m, a.cmax[h * a.max_chunks + c]);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        if (lane == 0) hinfo[wid] = m;
    }
    lds_barrier();
    // e_t
    for (int hh = 0; hh < kvm; ++hh) {
        const float M = hinfo[hh];
        const bool fin = __builtin_isfinite(M);
        const float *sc = a.scores + (size_t)(kvh * kvm + hh) * a.max_seq;
        for (int t = tid; t < n; t += PV_THREADS) {
            const float v = sc[t];
            p[hh * a.max_seq + t] = (fin && v > -INFINITY) ? exp256(v - M) : 0.0f;
        }
    }
    lds_barrier();
    // sums and the fp32 inverse, one wave per head
    if (wid < kvm) {
        const float *ph = p + wid * a.max_seq;
        float ls = 0.0f;
        if (lane < 8) {
            int t = lane;
            for (; t + 8 * 16 <= nb; t += 8 * 16) {
                float v[16];
#pragma unroll
                for (int u = 0; u < 16; ++u) v[u] = ph[t + 8 * u];
#pragma unroll
                for (int u = 0; u < 16; ++u) ls = ls + v[u];
            }
            for (; t < nb; t += 8) ls = ls + ph[t];
        }
        double sum = 0.0;
#pragma unroll
        for (int l = 0; l < 8; ++l) sum += (double)readlane_f(ls, l);
        for (int t = nb; t < n; ++t) sum += (double)ph[t];
        const bool ok = __builtin_isfinite(hinfo[wid]) && sum > 0.0 && __builtin_isfinite(sum);
        const float inv = ok ? (float)(1.0 / sum) : 0.0f;
        if (lane == 0) hinv[wid] = inv;
    }
    lds_barrier();
    for (int hh = 0; hh < kvm; ++hh) {
        const float inv = hinv[hh];
        for (int t = tid; t < n; t += PV_THREADS) p[hh * a.max_seq + t] *= inv;
    }

    // value-weighted sums
    const int ch_d = tid % PV_D, ch_h = tid / PV_D;
    const bool chain = ch_h < kvm;
    float acc = 0.0f;
    for (int t0 = 0; t0 < n; t0 += PV_TC) {
        lds_barrier();  // vt free (previous chains done); p final
        store_chunk();
        lds_barrier();
        if (t0 + PV_TC < n) load_chunk(t0 + PV_TC);
        if (chain) {
            const float *ph = p + ch_h * a.max_seq + t0;
            const uint32_t *vr = vt + ch_d * PV_RS;
            const int len = min(PV_TC, n - t0);
            // batches of 32 positions; the next batch's LDS reads are issued
            // before the current batch's FMAs (every read stays below len)
            auto fma8 = [&](const u32x4 &vv, const float4 &pa, const float4 &pb) {
                acc = fmaf(pa.x, h2f((uint16_t)vv.x), acc);
                acc = fmaf(pa.y, h2f((uint16_t)(vv.x >> 16)), acc);
                acc = fmaf(pa.z, h2f((uint16_t)vv.y), acc);
                acc = fmaf(pa.w, h2f((uint16_t)(vv.y >> 16)), acc);
                acc = fmaf(pb.x, h2f((uint16_t)vv.z), acc);
                acc = fmaf(pb.y, h2f((uint16_t)(vv.z >> 16)), acc);
                acc = fmaf(pb.z, h2f((uint16_t)vv.w), acc);
                acc = fmaf(pb.w, h2f((uint16_t)(vv.w >> 16)), acc);
            };
            int t = 0;
            if (len >= 32) {
                u32x4 cv[4];
                float4 cp[8];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    cv[u] = *reinterpret_cast<const u32x4 *>(vr + 4 * u);
                    cp[2 * u] = *reinterpret_cast<const float4 *>(ph + 8 * u);
                    cp[2 * u + 1] = *reinterpret_cast<const float4 *>(ph + 8 * u + 4);
                }
                for (; t + 32 <= len; t += 32) {
                    // next batch, or the last in-range batch (a multiple of 8)
                    const int tn = min(t + 32, (len - 32) & ~7);
                    u32x4 nv[4];
                    float4 np[8];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        nv[u] = *reinterpret_cast<const u32x4 *>(vr + tn / 2 + 4 * u);
                        np[2 * u] = *reinterpret_cast<const float4 *>(ph + tn + 8 * u);
                        np[2 * u + 1] = *reinterpret_cast<const float4 *>(ph + tn + 8 * u + 4);
                    }
#pragma unroll
                    for (int u = 0; u < 4; ++u) fma8(cv[u], cp[2 * u], cp[2 * u + 1]);
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        cv[u] = nv[u];
                        cp[2 * u] = np[2 * u];
                        cp[2 * u + 1] = np[2 * u + 1];
                    }
                }
            }
            for (; t + 8 <= len; t += 8) {
                const u32x4 vv = *reinterpret_cast<const u32x4 *>(vr + t / 2);
                fma8(vv, *reinterpret_cast<const float4 *>(ph + t),
                     *reinterpret_cast<const float4 *>(ph + t + 4));
            }
            for (; t < len; ++t) {
                const uint32_t w2 = vr[t / 2];
                acc = fmaf(ph[t], h2f((uint16_t)(w2 >> (16 * (t & 1)))), acc);
            }
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

hipError_t launch_rmsnorm_i8(const float *x, const int8_t *w, const float *ws, float *out, int n,
                             int gs, float eps, hipStream_t st) {
    if (n < 8 || n > RMS_MAX || n % 8 != 0 || gs <= 0 || n % gs != 0) return hipErrorInvalidValue;
    rmsnorm_i8_kernel<<<1, 256, 0, st>>>(x, w, ws, out, n, gs, eps);
    return hipGetLastError();
}

size_t attention_lds_bytes(int heads, int kv_heads, int max_seq) {
    return (size_t)PV_D * PV_RS * 4 + (size_t)(heads / kv_heads) * max_seq * 4;
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
