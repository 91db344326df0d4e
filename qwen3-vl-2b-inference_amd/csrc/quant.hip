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

}  // namespace q3vl
