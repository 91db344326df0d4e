// quant.hip -- per-row, per-group RMS activation quantizer (gfx950).
//
// Restates the reference quantizer of matmul/src/cpu_f32a_i8f32sb_f32c_avx2.cpp
// :135-177 (identical at :348-390 and :488-530) bit for bit:
//   sumsq: lane i of the 16 lanes of a group runs the FMA chain over
//          x[16t+i]^2, t = 0..gs/16-1 (the two 8-lane AVX accumulators), then
//          the fixed tree (v_i+v_{i+8}) -> +4 -> +1 -> +2 (simd_utils.hpp:5-19);
//   s    = sqrt(sumsq/gs + 1e-6) * fp32(1/127);  q = rne(x * fp32(1/s)),
//          saturated to int16.
// One group is handled by 16 lanes; a 256-thread block covers 16 groups.
#include "q3vl_device.hpp"
#include "q3vl_kernels.hpp"

namespace q3vl {

template <int GS, typename OutT>
__global__ __launch_bounds__(256) void quantize_rows_kernel(
    const float *__restrict__ A, OutT *__restrict__ q, float *__restrict__ a_s,
    int K, int ldq, int as_sm, int as_sg) {
    constexpr int T = GS / 16;
    const int Kg = K / GS;
    const int lane16 = threadIdx.x & 15;
    const int g = blockIdx.x * 16 + (threadIdx.x >> 4);
    const int m = blockIdx.y;
    const bool active = g < Kg;
    const float *x = A + (size_t)m * K + (size_t)(active ? g : 0) * GS;

    float v[T];
    float p = 0.0f;
#pragma unroll
    for (int t = 0; t < T; ++t) {
        v[t] = x[16 * t + lane16];
        p = fmaf(v[t], v[t], p);
    }
    // Lane i holds chain P0[i] (i<8) or P1[i-8] (i>=8). The xor-8, xor-4,
    // xor-1, xor-2 butterfly reproduces add_reduce_mm_256(P0+P1) exactly: each
    // step adds the same two operands as the AVX tree (fp32 add commutes).
    p = p + __shfl_xor(p, 8, 16);
    p = p + __shfl_xor(p, 4, 16);
    p = p + __shfl_xor(p, 1, 16);
    p = p + __shfl_xor(p, 2, 16);
    const float s = group_scale(p, 1.0f / (float)GS);
    const float inv = rcp_rn(s);
    if (!active) return;
    if (lane16 == 0) a_s[(size_t)m * as_sm + (size_t)g * as_sg] = s;
    OutT *qr = q + (size_t)m * ldq + (size_t)g * GS;
#pragma unroll
    for (int t = 0; t < T; ++t) qr[16 * t + lane16] = (OutT)quant_cvt(v[t] * inv);
}

template <typename OutT>
static hipError_t launch_quant(const float *A, OutT *q, float *a_s, int M, int K,
                               int gs, int ldq, int as_sm, int as_sg, hipStream_t st) {
    const int Kg = K / gs;
    dim3 grid((Kg + 15) / 16, M);
    switch (gs) {
#define Q3VL_QCASE(G)                                                              \
    case G:                                                                        \
        quantize_rows_kernel<G, OutT><<<grid, 256, 0, st>>>(A, q, a_s, K, ldq, as_sm, as_sg);   \
        break;
        Q3VL_QCASE(16) Q3VL_QCASE(32) Q3VL_QCASE(64) Q3VL_QCASE(128) Q3VL_QCASE(256)
#undef Q3VL_QCASE
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_quantize_i16(const float *A, int16_t *q, float *a_s, int M, int K,
                               int gs, hipStream_t st) {
    return launch_quant<int16_t>(A, q, a_s, M, K, gs, K, K / gs, 1, st);
}

hipError_t launch_quantize_f16(const float *A, _Float16 *q, float *a_sT, int M, int K,
                               int gs, int ldq, int lda_s, hipStream_t st) {
    return launch_quant<_Float16>(A, q, a_sT, M, K, gs, ldq, 1, lda_s, st);
}

// ------------------------------------------------ exporter weight quantizer
// quantize_groupwise (export_bin/export_qwen_bin.py:260-275) in numpy's fp32
// arithmetic: m = max|x| + 1e-8, s = m / 127, q = round half to even of
// x / s, clipped to [-127, 127] (|x / s| <= 127 (1 + 2^-24) for finite x, so
// no value is clipped and the int8 cast is exact). The values are finite, as
// the exporter's are.
//
// s is the IEEE fp32 quotient (div_rn). x / s is computed per element from
// r = RN(1/s) with two residual corrections (div_q below), which gives the
// IEEE quotient whenever it is >= 2^-80 in magnitude: the first correction
// makes the estimate faithful, the second is then correctly rounded
// (Markstein's theorem: r correctly rounded, faithful estimate, exact
// fma residual). Below 2^-80 the residual may underflow, and both quotients
// round to the integer 0, so q is always the exporter's.
Q3VL_INLINE float div_q(float x, float s, float r) {
    const float y0 = x * r;
    const float y1 = fmaf(fmaf(-s, y0, x), r, y0);
    return fmaf(fmaf(-s, y1, x), r, y1);
}

typedef float fx4 __attribute__((ext_vector_type(4)));

Q3VL_INLINE uint32_t quant4(fx4 v, float s, float r) {
    auto one = [&](float x) {
        const float t = fminf(fmaxf(__builtin_rintf(div_q(x, s, r)), -127.0f), 127.0f);
        return (uint32_t)(uint8_t)(int8_t)t;
    };
    return one(v.x) | (one(v.y) << 8) | (one(v.z) << 16) | (one(v.w) << 24);
}

Q3VL_INLINE float absmax4(fx4 v) {
    return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
}

// Groups of G <= 256 values (a power of two >= 4): G/4 lanes share a group,
// one float4 per lane, so a wave covers 256 consecutive values (a "chunk")
// per pass and U chunks are in flight per loop iteration.
template <int G, int U>
__global__ __launch_bounds__(256) void quantize_export_vec_kernel(const fx4 *__restrict__ x,
                                                                  size_t n4,
                                                                  uint32_t *__restrict__ q,
                                                                  float *__restrict__ scales) {
    constexpr int L = G / 4;
    const int lane = threadIdx.x & 63;
    const size_t wave = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const size_t nwaves = ((size_t)gridDim.x * blockDim.x) >> 6;
    for (size_t c0 = wave * U; c0 * 64 < n4; c0 += nwaves * U) {
        fx4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const size_t i = (c0 + u) * 64 + lane;
            v[u] = i < n4 ? __builtin_nontemporal_load(x + i) : fx4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const size_t i = (c0 + u) * 64 + lane;
            float m = absmax4(v[u]);
#pragma unroll
            for (int off = L / 2; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
            const float s = div_rn(m + 1e-8f, 127.0f);
            const float r = rcp_rn(s);
            if (i < n4) {  // n4 is a multiple of L: a group is wholly in or out
                if ((lane & (L - 1)) == 0) scales[i / L] = s;
                q[i] = quant4(v[u], s, r);
            }
        }
    }
}

// Groups of G > 256 values, G a multiple of 4: one wave per group; the max
// pass and the quantize pass each stream the group's float4s (the second
// read is an L2 hit for groups up to a few KB).
__global__ __launch_bounds__(256) void quantize_export_wave_kernel(const fx4 *__restrict__ x,
                                                                   size_t ngroups, int G4,
                                                                   uint32_t *__restrict__ q,
                                                                   float *__restrict__ scales) {
    const int lane = threadIdx.x & 63;
    const size_t wave = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const size_t nwaves = ((size_t)gridDim.x * blockDim.x) >> 6;
    for (size_t g = wave; g < ngroups; g += nwaves) {
        const fx4 *xg = x + g * (size_t)G4;
        float m0 = 0.0f, m1 = 0.0f;
        int i = lane;
        for (; i + 64 < G4; i += 128) {
            m0 = fmaxf(m0, absmax4(xg[i]));
            m1 = fmaxf(m1, absmax4(xg[i + 64]));
        }
        if (i < G4) m0 = fmaxf(m0, absmax4(xg[i]));
        float m = fmaxf(m0, m1);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        const float s = div_rn(m + 1e-8f, 127.0f);
        const float r = rcp_rn(s);
        if (lane == 0) scales[g] = s;
        uint32_t *qg = q + g * (size_t)G4;
        for (int j = lane; j < G4; j += 64) qg[j] = quant4(xg[j], s, r);
    }
}

// Any other group size or alignment: W lanes (a power of two, W <= group,
// W <= 64) share a group, one value per lane per step.
__global__ __launch_bounds__(256) void quantize_export_kernel(const float *__restrict__ x,
                                                              size_t ngroups, int group, int W,
                                                              int8_t *__restrict__ q,
                                                              float *__restrict__ scales) {
    const int lane = threadIdx.x & 63;
    const int sub = lane & (W - 1);
    const int per_wave = 64 / W;
    const size_t wave = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const size_t nwaves = ((size_t)gridDim.x * blockDim.x) >> 6;
    for (size_t g0 = wave * per_wave; g0 < ngroups; g0 += nwaves * per_wave) {
        const size_t gi = g0 + lane / W;
        const bool active = gi < ngroups;
        const float *xg = x + (active ? gi : 0) * (size_t)group;
        float m = 0.0f;
        if (active)
            for (int i = sub; i < group; i += W) m = fmaxf(m, fabsf(xg[i]));
        for (int off = W >> 1; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        const float s = div_rn(m + 1e-8f, 127.0f);
        const float r = rcp_rn(s);
        if (!active) continue;
        if (sub == 0) scales[gi] = s;
        int8_t *qg = q + gi * (size_t)group;
        for (int i = sub; i < group; i += W)
            qg[i] = (int8_t)fminf(fmaxf(__builtin_rintf(div_q(xg[i], s, r)), -127.0f), 127.0f);
    }
}

static unsigned grid_for(size_t waves) {
    const size_t blocks = (waves + 3) / 4;  // 4 waves per block
    return (unsigned)(blocks < (1u << 20) ? blocks : (1u << 20));
}

hipError_t launch_quantize_export(const float *x, size_t count, size_t group, int8_t *q,
                                  float *scales, hipStream_t st) {
    if (group == 0 || count % group != 0 || group > (size_t)INT32_MAX) return hipErrorInvalidValue;
    const size_t ngroups = count / group;
    if (ngroups == 0) return hipSuccess;
    const bool vec = group % 4 == 0 && ((uintptr_t)x & 15u) == 0 && ((uintptr_t)q & 3u) == 0;
    if (vec && group <= 256 && (group & (group - 1)) == 0) {
        constexpr int U = 2;
        const size_t n4 = count / 4;
        const size_t waves = ((n4 + 63) / 64 + U - 1) / U;
        const fx4 *x4 = reinterpret_cast<const fx4 *>(x);
        uint32_t *q4 = reinterpret_cast<uint32_t *>(q);
        switch (group) {
#define Q3VL_XCASE(G)                                                                       \
    case G:                                                                                 \
        quantize_export_vec_kernel<G, U><<<grid_for(waves), 256, 0, st>>>(x4, n4, q4, scales); \
        return hipGetLastError();
            Q3VL_XCASE(4) Q3VL_XCASE(8) Q3VL_XCASE(16) Q3VL_XCASE(32) Q3VL_XCASE(64)
            Q3VL_XCASE(128) Q3VL_XCASE(256)
#undef Q3VL_XCASE
        }
    }
    if (vec && group > 256) {
        quantize_export_wave_kernel<<<grid_for(ngroups), 256, 0, st>>>(
            reinterpret_cast<const fx4 *>(x), ngroups, (int)(group / 4),
            reinterpret_cast<uint32_t *>(q), scales);
        return hipGetLastError();
    }
    int W = 64;
    while ((size_t)W > group) W >>= 1;
    const size_t waves = (ngroups + (64 / W) - 1) / (64 / W);
    quantize_export_kernel<<<grid_for(waves), 256, 0, st>>>(x, ngroups, (int)group, W, q, scales);
    return hipGetLastError();
}

}  // namespace q3vl
