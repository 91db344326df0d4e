// hip_wrapper.cpp -- the engine's linear() over libq3vl_int8.so.
//
// Mirrors the dispatch of the reference's linear() (matmul/src/cpu_wrapper.cpp:
// 308-396): the int8 group-quantized branch (:339-348) runs on the GPU; other
// combinations go to linear_cpu_fallback() if the engine provides it, else the
// reference's "DType matmul not supported" message and exit(1) (:394-395).
#include "../include/hip_wrapper.hpp"

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <mutex>

#include "q3vl_int8.h"

namespace {

bool is_device_ptr(const void *p) {
    if (!p) return false;
    hipPointerAttribute_t attr{};
    const hipError_t e = hipPointerGetAttributes(&attr, p);
    if (e != hipSuccess) {
        (void)hipGetLastError();  // host pointers unknown to HIP report an error
        return false;
    }
    return attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged;
}

[[noreturn]] void die(const char *what) {
    fprintf(stderr, "linear (MI355X int8): %s\n", what);
    exit(1);
}

// Grow-only device staging for host activations / outputs.
struct Staging {
    std::mutex mu;
    void *a = nullptr;
    size_t a_bytes = 0;
    void *c = nullptr;
    size_t c_bytes = 0;
} g_stage;

void *grow(void *&p, size_t &have, size_t need) {
    if (need <= have) return p;
    if (p) (void)hipFree(p);
    p = nullptr;
    have = 0;
    if (hipMalloc(&p, need) != hipSuccess) die("staging hipMalloc failed");
    have = need;
    return p;
}

}  // namespace

void linear(const void *mat_A, const void *mat_B_in, const void *mat_B_scale,
            const void *mat_bias_in, const void *mat_bias_scale, void *mat_C, size_t M,
            size_t N, size_t K, bool mat_B_transpose, DType::Type type_a,
            DType::Type type_b, DType::Type type_b_scale, DType::Type type_c,
            bool group_quantized, size_t group_size) {
    if (q3vl_check_dtypes((int)type_a, (int)type_b, (int)type_b_scale, (int)type_c,
                          mat_bias_in != nullptr, group_quantized, mat_B_transpose) != Q3VL_OK) {
        if (linear_cpu_fallback) {
            linear_cpu_fallback(mat_A, mat_B_in, mat_B_scale, mat_bias_in, mat_bias_scale, mat_C,
                                M, N, K, mat_B_transpose, type_a, type_b, type_b_scale, type_c,
                                group_quantized, group_size);
            return;
        }
        fprintf(stderr, "%s\n", q3vl_last_error());
        exit(1);
    }
    if (M == 0 || N == 0) return;

    // Weights: device pointers pass through; host weights (mmapped by the
    // engine's loader) are uploaded once and found again by host address,
    // scale address, shape and a fingerprint of their bytes; a stale entry
    // (another weight at the same address) is replaced by registering again.
    const int8_t *dW = static_cast<const int8_t *>(mat_B_in);
    const float *dS = static_cast<const float *>(mat_B_scale);
    if (!is_device_ptr(mat_B_in)) {
        if (q3vl_weight_lookup(mat_B_in, static_cast<const float *>(mat_B_scale), N, K,
                               group_size, &dW, &dS) != Q3VL_OK &&
            q3vl_weight_register(static_cast<const int8_t *>(mat_B_in),
                                 static_cast<const float *>(mat_B_scale), N, K, group_size, &dW,
                                 &dS) != Q3VL_OK)
            die(q3vl_last_error());
    }

    std::lock_guard<std::mutex> lk(g_stage.mu);
    const float *dA = static_cast<const float *>(mat_A);
    if (!is_device_ptr(mat_A)) {
        void *p = grow(g_stage.a, g_stage.a_bytes, M * K * sizeof(float) + 16);
        if (hipMemcpy(p, mat_A, M * K * sizeof(float), hipMemcpyHostToDevice) != hipSuccess)
            die("activation upload failed");
        dA = static_cast<const float *>(p);
    }
    const bool c_host = !is_device_ptr(mat_C);
    float *dC = static_cast<float *>(mat_C);
    if (c_host) dC = static_cast<float *>(grow(g_stage.c, g_stage.c_bytes, M * N * sizeof(float)));

    if (q3vl_linear_i8(dA, dW, dS, dC, M, N, K, group_size, nullptr, 0, nullptr) != Q3VL_OK)
        die(q3vl_last_error());
    if (c_host) {
        if (hipMemcpy(mat_C, dC, M * N * sizeof(float), hipMemcpyDeviceToHost) != hipSuccess)
            die("result download failed");
    } else if (hipStreamSynchronize(nullptr) != hipSuccess) {
        die("hipStreamSynchronize failed");
    }
}
