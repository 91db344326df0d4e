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
#include <cstring>

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

// Grow-only staging for host activations and outputs, one set per calling
// thread (no lock): pinned host buffers, so that the copies are asynchronous
// DMA on the call's stream and the call waits once, and device buffers.
struct Staging {
    void *ha = nullptr, *hc = nullptr;  // pinned host
    size_t ha_bytes = 0, hc_bytes = 0;
    void *da = nullptr, *dc = nullptr;  // device
    size_t da_bytes = 0, dc_bytes = 0;
    ~Staging() {
        if (ha) (void)hipHostFree(ha);
        if (hc) (void)hipHostFree(hc);
        if (da) (void)hipFree(da);
        if (dc) (void)hipFree(dc);
    }
};
thread_local Staging t_stage;

void *grow_device(void *&p, size_t &have, size_t need) {
    if (need <= have) return p;
    if (p) (void)hipFree(p);
    p = nullptr;
    have = 0;
    if (hipMalloc(&p, need) != hipSuccess) die("staging hipMalloc failed");
    have = need;
    return p;
}

void *grow_pinned(void *&p, size_t &have, size_t need) {
    if (need <= have) return p;
    if (p) (void)hipHostFree(p);
    p = nullptr;
    have = 0;
    if (hipHostMalloc(&p, need, hipHostMallocDefault) != hipSuccess) die("staging hipHostMalloc failed");
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

    // Host activations and outputs go through this thread's pinned staging:
    // upload, kernel and download are queued on the null stream (ordered
    // after the engine's own device work, as the synchronous copies were) and
    // the call waits once.
    Staging &st = t_stage;
    const size_t a_bytes = M * K * sizeof(float), c_bytes = M * N * sizeof(float);
    const float *dA = static_cast<const float *>(mat_A);
    if (!is_device_ptr(mat_A)) {
        void *h = grow_pinned(st.ha, st.ha_bytes, a_bytes);
        void *d = grow_device(st.da, st.da_bytes, a_bytes + 16);
        memcpy(h, mat_A, a_bytes);
        if (hipMemcpyAsync(d, h, a_bytes, hipMemcpyHostToDevice, nullptr) != hipSuccess)
            die("activation upload failed");
        dA = static_cast<const float *>(d);
    }
    // A host C of a GEMV (M <= 8: at most 8 rows) is written by the kernel
    // straight into the pinned buffer (device-accessible host memory), with
    // no download; a larger one goes through a device buffer and a copy.
    const bool c_host = !is_device_ptr(mat_C);
    const bool c_direct = c_host && M <= 8;
    float *dC = static_cast<float *>(mat_C);
    void *hc = nullptr;
    if (c_host) hc = grow_pinned(st.hc, st.hc_bytes, c_bytes);
    if (c_direct) {
        void *p = nullptr;
        if (hipHostGetDevicePointer(&p, hc, 0) != hipSuccess) die("hipHostGetDevicePointer failed");
        dC = static_cast<float *>(p);
    } else if (c_host) {
        dC = static_cast<float *>(grow_device(st.dc, st.dc_bytes, c_bytes));
    }

    if (q3vl_linear_i8(dA, dW, dS, dC, M, N, K, group_size, nullptr, 0, nullptr) != Q3VL_OK)
        die(q3vl_last_error());
    if (c_host && !c_direct &&
        hipMemcpyAsync(hc, dC, c_bytes, hipMemcpyDeviceToHost, nullptr) != hipSuccess)
        die("result download failed");
    if (hipStreamSynchronize(nullptr) != hipSuccess) die("hipStreamSynchronize failed");
    if (c_host) memcpy(mat_C, hc, c_bytes);
}
