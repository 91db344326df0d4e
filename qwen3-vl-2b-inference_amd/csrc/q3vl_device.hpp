// q3vl_device.hpp -- device helpers shared by the int8 matmul kernels (gfx950).
//
// Numerics follow the reference's AVX2 int8 path
// (matmul/src/cpu_f32a_i8f32sb_f32c_avx2.cpp, matmul/include/simd_utils.hpp).
// All kernels are compiled with -ffp-contract=off: every fused multiply-add is
// written as fmaf(), every other operation rounds on its own.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <cfloat>

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

// The same for two values, packed as int16 (lo in bits 0..15): the int32 of
// cvtps2dq is INT32_MIN exactly when !(|p| < 2^31) (NaN, overflow, and
// p = -2^31 itself, where the rounded value is INT32_MIN anyway), and
// v_cvt_pk_i16_i32 applies packs_epi32's signed saturation to both.
Q3VL_INLINE uint32_t quant_pair(float lo, float hi) {
    const int32_t a = __builtin_fabsf(lo) < 2147483648.0f ? (int32_t)__builtin_rintf(lo) : INT32_MIN;
    const int32_t b = __builtin_fabsf(hi) < 2147483648.0f ? (int32_t)__builtin_rintf(hi) : INT32_MIN;
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pk_i16(a, b));
}

// quant_pair for a group whose scale s is finite. Then every x of the group
// was finite with x^2 <= the group's sum of squares, so |x / s| <= 127 *
// sqrt(gs) * (1 + 2^-16) < 2^22: adding 1.5 * 2^23 rounds to the nearest
// integer, ties to even (the sum lies in [2^23, 2^24), whose spacing is 1),
// and the integer is the sum's bits less the constant's. Equal to
// quant_pair there (its INT32_MIN cases need a non-finite q).
Q3VL_INLINE uint32_t quant_pair_finite(float lo, float hi) {
    constexpr float kMagic = 12582912.0f;  // 1.5 * 2^23
    constexpr int32_t kMagicBits = 0x4B400000;
    const int32_t a = __builtin_bit_cast(int32_t, lo + kMagic) - kMagicBits;
    const int32_t b = __builtin_bit_cast(int32_t, hi + kMagic) - kMagicBits;
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pk_i16(a, b));
}

// Correctly rounded fp32 sqrt and reciprocal. sqrt: the compiler's IEEE
// expansion of the fp32 square root (hardware estimate, then a one-ulp
// correction from fma residuals), about 15 fp32 operations; it equals the
// double-precision root rounded once to fp32 for every non-negative fp32
// input (compared exhaustively on the device), at half the latency of the
// fp64 sequence. Reciprocal and division: computed in double and rounded
// once; for division the double rounding is innocuous (53 >= 2*24+2), so the
// result equals the IEEE fp32 operation (and compiles to the fp32 one).
Q3VL_INLINE float sqrt_rn(float x) { return __builtin_sqrtf(x); }
Q3VL_INLINE float rcp_rn(float x) { return (float)(1.0 / (double)x); }
Q3VL_INLINE float div_rn(float a, float b) { return (float)((double)a / (double)b); }

// expf as the reference's host libm computes it (glibc >= 2.27 uses the
// ARM optimized-routines expf by Szabolcs Nagy; on x86-64 CPUs with FMA the
// ifunc selects the build of it compiled with FMA contraction). With N = 32:
//   x*N/ln2 = k + r (k rounded to nearest via the 1.5*2^52 shift),
//   exp(x) = 2^(k/N) * (1 + C2 r + C1 r^2 + C0 r^3) evaluated in double,
// every multiply that feeds an add fused into an fma, as the compiler does.
// kExp2Tab32[i] = bits(double nearest 2^(i/32)) - (i << 47); adding k << 47
// to an entry applies 2^floor(k/32). Rounded once to fp32 at the end. This
// equals the host's expf on every one of the 2^32 inputs (checked
// exhaustively on the CPU against glibc 2.35's expf).
static __constant__ uint64_t kExp2Tab32[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

Q3VL_INLINE float expf_host(float x) {
    if (x != x) return x + x;
    if (x > 0x1.62e42ep6f) return __builtin_inff();
    if (x < -0x1.9fe368p6f) return 0.0f;
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0);
    const double c1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0);
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    double kd = __builtin_fma(inv_ln2_n, xd, shift);
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd = kd - shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    const double s = __builtin_bit_cast(double, kExp2Tab32[ki & 31] + (ki << 47));
    const double z = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    const double y = __builtin_fma(c2, r, 1.0);
    return (float)(__builtin_fma(z, r2, y) * s);
}

// SwiGLU element, layers/src/text_layer.cpp:428-433: silu = g / (1 + expf(-g)),
// h = silu * u; the fp32 division is correctly rounded (double quotient
// rounded once: innocuous, 53 >= 2*24+2).
Q3VL_INLINE float silu_mul(float gv, float uv) {
    const float den = 1.0f + expf_host(-gv);
    const float sl = (float)((double)gv / (double)den);
    return sl * uv;
}

// Combine rule equivalent to the sequential strict-> scan of greedy_decode:
// the larger value wins, equal values keep the lower index, idx<0 is empty.
__device__ __forceinline__ void am_combine(float &bv, int32_t &bi, float v, int32_t i) {
    if (i < 0) return;
    if (bi < 0 || v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

// Workgroup barrier that orders LDS only: global loads stay in flight across
// it (a full __syncthreads() waits for every outstanding global access).
Q3VL_INLINE void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

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

// dot2(a, b, 0) as one VOP3P instruction with an inline 0 accumulator (the
// compiler picks the two-operand form, whose accumulator a move must zero).
Q3VL_INLINE int32_t dot2_z(uint32_t a, uint32_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
    int32_t r;
    asm("v_dot2_i32_i16 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
#else
    return dot2(a, b, 0);
#endif
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

// One step of scatter_sums over n values: the thread keeps the half of
// v[0..n) its final sums lie in (the upper half when hi) and adds the
// partner's copy of that half; with one value left both add it whole.
template <int n, int N, typename Dpp>
Q3VL_INLINE void scatter_step(int32_t (&v)[N], bool hi, Dpp dpp) {
    if constexpr (n == 1) {
        v[0] += dpp(v[0]);
    } else {
        constexpr int H = n / 2;
#pragma unroll
        for (int k = 0; k < H; ++k) {
            const int32_t keep = hi ? v[H + k] : v[k];
            const int32_t send = hi ? v[k] : v[H + k];
            v[k] = keep + dpp(send);
        }
    }
}

// Reduce-scatter of N per-thread sums (N = 1, 2, 4 or 8) over the aligned
// run of T threads (T = 1, 2, 4 or 8) that holds one group. When N >= T,
// thread tg of the run ends with the run's totals for sums
// j = tg*W .. tg*W + W-1 (W = N/T) in v[0..W); when N < T, with the total
// for sum j = tg / (T/N) in v[0], which the T/N threads tg of that sum all
// hold. Each step halves the set by one bit of tg (bit 2 against the half
// mirror, bit 1 against xor 2, bit 0 against xor 1), highest bit first.
// Integer adds, so the totals equal any other summation order.
template <int T, int N>
Q3VL_INLINE void scatter_sums(int32_t (&v)[N], int tg) {
    static_assert(T == 1 || T == 2 || T == 4 || T == 8, "group run of 1, 2, 4 or 8 threads");
    static_assert(N == 1 || N == 2 || N == 4 || N == 8, "1, 2, 4 or 8 sums");
    // every index is a compile-time constant (a select over a run-time
    // index would become compare chains)
    constexpr int n2 = N;
    constexpr int n1 = T == 8 ? (n2 > 1 ? n2 / 2 : 1) : n2;
    constexpr int n0 = T >= 4 ? (n1 > 1 ? n1 / 2 : 1) : n1;
    if constexpr (T == 8) scatter_step<n2>(v, (tg & 4) != 0, [](int32_t x) { return dpp_half_mirror(x); });
    if constexpr (T >= 4) scatter_step<n1>(v, (tg & 2) != 0, [](int32_t x) { return dpp_xor2(x); });
    if constexpr (T >= 2) scatter_step<n0>(v, (tg & 1) != 0, [](int32_t x) { return dpp_xor1(x); });
}

}  // namespace q3vl
