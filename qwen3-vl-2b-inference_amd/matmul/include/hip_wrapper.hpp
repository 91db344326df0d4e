// hip_wrapper.hpp -- the engine's matmul entry points, unchanged signatures
// (matmul/include/cpu_wrapper.hpp:10-21 of the reference engine).
//
// linear(): the int8 group-quantized combination (FP32 A, INT8 B with FP32
// group scales, FP32 C, no bias, B transposed) runs on the MI355X through the
// C ABI in include/q3vl_int8.h. Any other combination is forwarded to
// linear_cpu_fallback() when the engine links its CPU matmul sources under
// that name; without it the call fails like the reference's unsupported
// combination (fprintf + exit(1), matmul/src/cpu_wrapper.cpp:394-395).
//
// Contract kept from the reference: synchronous (C is complete on return),
// C overwritten, caller owns all buffers. A, B, B_scale and C may be host or
// device pointers; host weights are uploaded once through the library's
// weight registry and reused on later calls with the same host address.
#pragma once

#include <cstddef>
#include <cstdint>

#include "../../utils/module.hpp"

void linear(const void *mat_A, const void *mat_B_in, const void *mat_B_scale,
            const void *mat_bias_in, const void *mat_bias_scale, void *mat_C, size_t M,
            size_t N, size_t K, bool mat_B_transpose, DType::Type type_a,
            DType::Type type_b, DType::Type type_b_scale, DType::Type type_c,
            bool group_quantized, size_t group_size);

// Declared for source compatibility; defined by the engine's CPU matmul
// sources (vision attention, not on the int8 path).
void gemm_att(const void *mat_A, const void *mat_B, void *mat_C, const float scale,
              size_t N, size_t K, bool mat_B_transpose, DType::Type type_a,
              DType::Type type_b, DType::Type type_c);

// Optional: the engine's original CPU linear(), compiled under this name
// (e.g. -Dlinear=linear_cpu_fallback on matmul/src/cpu_wrapper.cpp).
void linear_cpu_fallback(const void *mat_A, const void *mat_B_in, const void *mat_B_scale,
                         const void *mat_bias_in, const void *mat_bias_scale, void *mat_C,
                         size_t M, size_t N, size_t K, bool mat_B_transpose,
                         DType::Type type_a, DType::Type type_b, DType::Type type_b_scale,
                         DType::Type type_c, bool group_quantized, size_t group_size)
    __attribute__((weak));
