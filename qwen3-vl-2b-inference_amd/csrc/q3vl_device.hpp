// q3vl_device.hpp -- device helpers shared by the int8 matmul kernels (gfx950).
//
// Numerics follow the reference's AVX2 int8 path
// (matmul/src/cpu_f32a_i8f32sb_f32c_avx2.cpp, matmul/include/simd_utils.hpp).
// All kernels are compiled with -ffp-contract=off: every fused multiply-add is
// written as fmaf(), every other operation rounds on its own.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#ifndef Q3VL_INLINE
#define Q3VL_INLINE __device__ __forceinline__
#endif

namespace q3vl {

// Fixed fp32 reduction tree of add_reduce_mm_256 (simd_utils.hpp:5-19):
// ((v0+v4)+(v1+v5)) + ((v2+v6)+(v3+v7)).
Q3VL_INLINE float tree8(float v0, float v1, float v2, float v3, float v4,
                        float v5, float v6, float v7) {
    const float s0 = v0 + v4, s1 = v1 + v5, s2 = v2 + v6, s3 = v3 + v7;
    return (s0 + s1) + (s2 + s3);
}

// cvtps2dq under round-to-nearest-even: NaN / out of int32 range -> INT32_MIN,
// then packs_epi32 saturation to int16 (quantizer steps i8:164-175).
Q3VL_INLINE int32_t quant_cvt(float p) {
    int32_t v;
    if (!(p >= -2147483648.0f && p < 2147483648.0f)) v = INT32_MIN;
    else v = (int32_t)__builtin_rintf(p);
    v = v > 32767 ? 32767 : v;
    v = v < -32768 ? -32768 : v;
    return v;
}

// Correctly rounded fp32 sqrt and reciprocal: computed in double and rounded
// once to fp32. For sqrt and division the double rounding is innocuous
// (53 >= 2*24+2), so the result equals the IEEE fp32 operation.
Q3VL_INLINE float sqrt_rn(float x) { return (float)__builtin_sqrt((double)x); }
Q3VL_INLINE float rcp_rn(float x) { return (float)(1.0 / (double)x); }

// Group scale from the 16 per-lane partial sums of squares of one group
// (i8:148-152): the caller passes the sum tree already reduced; this applies
// rms = sqrt(sumsq/gs + 1e-6), s = rms * fp32(1/127).
Q3VL_INLINE float group_scale(float sumsq, float inv_gs) {
    const float rms = sqrt_rn(sumsq * inv_gs + 1e-6f);
    const float inv_127 = 1.0f / 127.0f;  // folded at compile time, as i8:130
    return rms * inv_127;
}

// Place the int8 bytes of one dword into the high byte of two int16 lanes:
// lo2(w) = (b0<<8, b1<<8), hi2(w) = (b2<<8, b3<<8). A v_dot2_i32_i16 against
// int16 activation pairs then yields 256x the exact pair product sum.
Q3VL_INLINE uint32_t lo2(uint32_t w) { return __builtin_amdgcn_perm(w, w, 0x010C000Cu); }
Q3VL_INLINE uint32_t hi2(uint32_t w) { return __builtin_amdgcn_perm(w, w, 0x030C020Cu); }

// v_dot2_i32_i16: a.lo*b.lo + a.hi*b.hi + c (signed 16-bit lanes).
typedef short short2_t __attribute__((ext_vector_type(2)));
Q3VL_INLINE int32_t dot2(uint32_t a, uint32_t b, int32_t c) {
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(short2_t, a),
                                  __builtin_bit_cast(short2_t, b), c, false);
}

// DPP sums inside a quad of lanes (row_mask/bank_mask all lanes).
// quad_perm [1,0,3,2] = 0xB1 (xor 1), [2,3,0,1] = 0x4E (xor 2).
Q3VL_INLINE int32_t dpp_xor1(int32_t v) {
    return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
}
Q3VL_INLINE int32_t dpp_xor2(int32_t v) {
    return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
}
// row_half_mirror (lane i <-> 7-i inside 8) and row_mirror (i <-> 15-i inside
// 16): after a full quad sum these complete 8- and 16-lane sums.
Q3VL_INLINE int32_t dpp_half_mirror(int32_t v) {
    return __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);
}
Q3VL_INLINE int32_t dpp_mirror(int32_t v) {
    return __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false);
}

// Sum of v over the aligned run of `width` lanes (1, 2, 4, 8 or 16) that
// contains this lane; every lane of the run receives the sum. Integer adds,
// so the order is immaterial.
template <int WIDTH>
Q3VL_INLINE int32_t run_sum(int32_t v) {
    if constexpr (WIDTH >= 2) v += dpp_xor1(v);
    if constexpr (WIDTH >= 4) v += dpp_xor2(v);
    if constexpr (WIDTH >= 8) v += dpp_half_mirror(v);
    if constexpr (WIDTH >= 16) v += dpp_mirror(v);
    return v;
}

}  // namespace q3vl
