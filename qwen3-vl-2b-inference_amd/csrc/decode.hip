// decode.hip -- support kernels of the text decode step that calls the int8
// path (model/src/forward.cpp:458-720), gfx950.
//
// Numerics follow the reference where its order is explicit (RoPE fmas,
// exp256_ps, the 8-lane attention dot products, fp16 KV stores) and the fixed
// orders of the CPU oracle where the reference leaves them to the compiler
// (RMS sum of squares). Attention normalizes with the exact global maximum
// (as the reference's softmax does) so exp256 sees the same arguments; only
// the softmax sum and the value-weighted sum are accumulated in a different
// (parallel) order.
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
__device__ __forceinline__ uint16_t f2h(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);  // round to nearest even
}

// Sum of squares of a 128-vector held as (lo = x[lane], hi = x[lane+64]) by
// one wave, in the oracle's fixed order: 128 one-element chains, then the
// binary tree p[c] += p[c+w], w = 64..1.
__device__ __forceinline__ float wave_sumsq128(float lo, float hi) {
    float v = fmaf(lo, lo, 0.0f) + fmaf(hi, hi, 0.0f);
#pragma unroll
    for (int w = 32; w >= 1; w >>= 1) v = v + __shfl_down(v, w);
    return __shfl(v, 0);
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
// One block of 256 threads per row. mode 0: rms_norm (text_layer.cpp:
// 110-147), inv = (float)(1/sqrt(double(ss/n + eps))); mode 1:
// rms_norm_inplace (text_layer.cpp:234-270), inv = 1.0f/sqrtf(ss/n + eps).
// out = w * ((s_g * inv) * x). Sum of squares in the oracle's fixed order:
// 256 chains (chain c: x[c], x[c+256], ...), then p[c] += p[c+w], w=128..1.
__global__ __launch_bounds__(256) void rmsnorm_i8_kernel(const float *x, const int8_t *w,
                                                         const float *ws, float *out, int n,
                                                         int gs, float eps, int mode) {
    __shared__ float p[256];
    __shared__ float s_inv;
    const int c = threadIdx.x;
    const int C = n < 256 ? n : 256;
    float v = 0.0f;
    if (c < C)
        for (int j = c; j < n; j += C) v = fmaf(x[j], x[j], v);
    p[c] = v;
    __syncthreads();
    for (int wdt = C / 2; wdt >= 64; wdt >>= 1) {
        if (c < wdt) p[c] = p[c] + p[c + wdt];
        __syncthreads();
    }
    if (c < 64) {
        float t = p[c];
        for (int wdt = (C / 2 < 32 ? C / 2 : 32); wdt >= 1; wdt >>= 1) t = t + __shfl_down(t, wdt);
        if (c == 0) {
            const float arg = t * (1.0f / (float)n) + eps;
            s_inv = mode == 0 ? (float)(1.0 / __builtin_sqrt((double)arg)) : rcp_rn(sqrt_rn(arg));
        }
    }
    __syncthreads();
    const float inv = s_inv;
    for (int j = c; j < n; j += 256) out[j] = (float)w[j] * ((ws[j / gs] * inv) * x[j]);
}

// --------------------------------------------------------------- attention
// A: per (kv head, chunk of ATT_CH positions), one wave per query head of the
// group. The waves normalize + rotate their query heads (q RMSNorm + RoPE,
// forward.cpp:531-545); the chunk holding `pos` also normalizes + rotates the
// new key and stores it and the new value as fp16 at pos (forward.cpp:
// 548-562). Scores follow text_layer.cpp:598-620 exactly: 8 FMA lane chains
// over the head dimension, the fixed tree, times 1/sqrt(hd).
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
        score = tree8(cc[0], cc[1], cc[2], cc[3], cc[4], cc[5], cc[6], cc[7]) * a.inv_sqrt_d;
        a.scores[(size_t)h * a.max_seq + t] = score;
    }
    float m = score;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if (lane == 0) a.cmax[h * a.max_chunks + ch] = m;
}

// B: per (query head, chunk): e_t = exp256(s_t - M) with the head's exact
// maximum M, chunk sum of e_t and partial value sums sum_t e_t * v_t[d].
__global__ __launch_bounds__(ATT_HD) void attn_pv_kernel(AttnArgs a) {
    __shared__ float e[ATT_CH];
    __shared__ float red[2];
    const int h = blockIdx.x, ch = blockIdx.y;
    const int pos = *a.pos;
    const int n = pos + 1;
    const int t0 = ch * ATT_CH;
    if (t0 >= n) return;
    const int nch = (n + ATT_CH - 1) / ATT_CH;
    const int d = threadIdx.x;
    const int kvm = a.heads / a.kv_heads;
    // exact maximum over the head's chunk maxima
    float M = -INFINITY;
    for (int c = 0; c < nch; ++c) M = fmaxf(M, a.cmax[h * a.max_chunks + c]);
    const int rows = min(ATT_CH, n - t0);
    if (d < ATT_CH) {
        float ev = 0.0f;
        if (d < rows) {
            const float sc = a.scores[(size_t)h * a.max_seq + t0 + d];
            ev = sc > -INFINITY ? exp256(sc - M) : 0.0f;  // text_layer.cpp:486-493
        }
        e[d] = ev;
        float sum = ev;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
        if (d == 0) red[0] = sum;
    }
    __syncthreads();
    const uint16_t *vc = a.v_cache + (size_t)a.layer * a.kv_heads * a.max_seq * ATT_HD +
                         ((size_t)(h / kvm) * a.max_seq + t0) * ATT_HD;
    float o = 0.0f;
#pragma unroll 8
    for (int r = 0; r < rows; ++r) o = fmaf(e[r], h2f(vc[(size_t)r * ATT_HD + d]), o);
    a.po[((size_t)h * a.max_chunks + ch) * ATT_HD + d] = o;
    if (d == 0) a.psum[h * a.max_chunks + ch] = red[0];
}

// C: per query head: sum = sum_c psum_c (double, chunk order), inv = 1/sum as
// in text_layer.cpp:522, out[d] = (sum_c po_c[d]) * inv. A head whose sum is
// not positive and finite gets zeros (text_layer.cpp:514-517).
__global__ __launch_bounds__(ATT_HD) void attn_combine_kernel(AttnArgs a) {
    const int h = blockIdx.x, d = threadIdx.x;
    const int pos = *a.pos;
    const int nch = (pos + 1 + ATT_CH - 1) / ATT_CH;
    double sum = 0.0;
    float o = 0.0f;
    for (int c = 0; c < nch; ++c) {
        sum += (double)a.psum[h * a.max_chunks + c];
        o += a.po[((size_t)h * a.max_chunks + c) * ATT_HD + d];
    }
    float r = 0.0f;
    if (sum > 0.0 && __builtin_isfinite(sum)) r = o * (float)(1.0 / sum);
    a.out[h * ATT_HD + d] = r;
}

// ------------------------------------------------------------------ launch
hipError_t launch_embed(const int8_t *w, const float *s, const int32_t *token, float *x, int H,
                        int gs, hipStream_t st) {
    embed_kernel<<<(H + 255) / 256, 256, 0, st>>>(w, s, token, x, H, gs);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_i8(const float *x, const int8_t *w, const float *ws, float *out, int n,
                             int gs, float eps, int mode, hipStream_t st) {
    if (n < 2 || (n & (n - 1)) != 0 || n % gs != 0) return hipErrorInvalidValue;
    rmsnorm_i8_kernel<<<1, 256, 0, st>>>(x, w, ws, out, n, gs, eps, mode);
    return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs &a, hipStream_t st) {
    const int kvm = a.heads / a.kv_heads;
    if (a.head_dim != ATT_HD || a.heads % a.kv_heads != 0 || kvm < 1 || kvm > 3)
        return hipErrorInvalidValue;
    attn_scores_kernel<<<dim3(a.kv_heads, a.max_chunks), 64 * (kvm + 1), 0, st>>>(a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    attn_pv_kernel<<<dim3(a.heads, a.max_chunks), ATT_HD, 0, st>>>(a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    attn_combine_kernel<<<a.heads, ATT_HD, 0, st>>>(a);
    return hipGetLastError();
}

}  // namespace q3vl
