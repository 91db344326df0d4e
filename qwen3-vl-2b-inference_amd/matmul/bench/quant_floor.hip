// quant_floor.hip -- what the stand-alone fragment-order quantizer ahead of
// each prefill / vision GEMM costs inside a replayed HIP graph, against the
// floor of its bytes:
//   * the quantizer alone, its fp32 input hot (one copy) and cold (copies
//     rotated over more than 640 MB), against a kernel that reads the same
//     fp32 bytes and writes half as many (the fp16 q);
//   * the quantizer followed by its GEMM against the GEMM alone, weights
//     rotated over 24 copies as a pass over the vision encoder's blocks
//     rotates them: the difference is what the quantizer adds in sequence.
// At config 4's vision shapes (784 tokens).
// One JSON object per line.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <vector>

#include "q3vl_kernels.hpp"

#define CHECK(x)                                                                             \
    do {                                                                                     \
        hipError_t e_ = (x);                                                                 \
        if (e_ != hipSuccess) {                                                              \
            fprintf(stderr, "quant_floor: %s at line %d\n", hipGetErrorString(e_), __LINE__); \
            return 1;                                                                        \
        }                                                                                    \
    } while (0)

// reads n4 float4 and writes one 8-byte value for each (half the bytes)
__global__ __launch_bounds__(256) void copy_half_kernel(const float4 *__restrict__ a, uint2 *__restrict__ q,
                                                        size_t n4) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n4) {
        const float4 v = a[i];
        q[i] = make_uint2(__float_as_uint(v.x + v.y), __float_as_uint(v.z + v.w));
    }
}

// best of 5 replays of a graph of `reps` calls of launch(r), in us per call
template <class F>
static int time_graph(hipStream_t st, int reps, F launch, float *us) {
    hipGraph_t g;
    hipGraphExec_t ge;
    CHECK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
    for (int r = 0; r < reps; ++r) CHECK(launch(r));
    CHECK(hipStreamEndCapture(st, &g));
    CHECK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
    CHECK(hipGraphLaunch(ge, st));
    CHECK(hipStreamSynchronize(st));
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    float best = 1e30f;
    for (int t = 0; t < 5; ++t) {
        CHECK(hipEventRecord(e0, st));
        CHECK(hipGraphLaunch(ge, st));
        CHECK(hipEventRecord(e1, st));
        CHECK(hipEventSynchronize(e1));
        float ms = 0.0f;
        CHECK(hipEventElapsedTime(&ms, e0, e1));
        best = ms * 1000.0f / reps < best ? ms * 1000.0f / reps : best;
    }
    CHECK(hipEventDestroy(e0));
    CHECK(hipEventDestroy(e1));
    CHECK(hipGraphExecDestroy(ge));
    CHECK(hipGraphDestroy(g));
    *us = best;
    return 0;
}

int main() {
    hipStream_t st;
    CHECK(hipStreamCreate(&st));
    int cus = 0;
    CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
    // M, N, K: vision qkv, proj, fc1, fc2
    const int shapes[][3] = {{784, 3072, 1024}, {784, 1024, 1024}, {784, 4096, 1024}, {784, 1024, 4096}};
    for (const auto &sh : shapes) {
        const int M = sh[0], N = sh[1], K = sh[2], Mt = (M + 31) / 32, NW = 24, reps = 96;
        const size_t na = (size_t)M * K;
        const int NA = (int)((640ull << 20) / (na * 4)) + 1;  // input copies: > 640 MB
        std::vector<float> ha(na);
        for (size_t i = 0; i < na; ++i) ha[i] = (float)((i * 2654435761u) % 2001) / 100.0f - 10.0f;
        std::vector<int8_t> hw((size_t)N * K);
        for (size_t i = 0; i < hw.size(); ++i) hw[i] = (int8_t)((int)((i * 40503u) % 255) - 127);
        std::vector<float> hs((size_t)N * K / 64, 0.01f);
        std::vector<float *> A(NA);
        for (auto &p : A) {
            CHECK(hipMalloc(&p, na * 4));
            CHECK(hipMemcpy(p, ha.data(), na * 4, hipMemcpyHostToDevice));
        }
        std::vector<int8_t *> W(NW);
        std::vector<float *> S(NW);
        for (int c = 0; c < NW; ++c) {
            CHECK(hipMalloc(&W[c], hw.size()));
            CHECK(hipMemcpy(W[c], hw.data(), hw.size(), hipMemcpyHostToDevice));
            CHECK(hipMalloc(&S[c], hs.size() * 4));
            CHECK(hipMemcpy(S[c], hs.data(), hs.size() * 4, hipMemcpyHostToDevice));
        }
        _Float16 *qf;
        float *as, *C;
        uint2 *cq;
        CHECK(hipMalloc(&qf, (size_t)Mt * 32 * K * 2));
        CHECK(hipMalloc(&as, (size_t)Mt * 32 * (K / 64) * 4));
        CHECK(hipMalloc(&C, (size_t)M * N * 4));
        CHECK(hipMalloc(&cq, na * 2));
        const size_t n4 = na / 4;
        const unsigned cgrid = (unsigned)((n4 + 255) / 256);
        auto quant = [&](int r) { return q3vl::launch_quantize_frag(A[r % NA], qf, as, M, K, st); };
        auto copy = [&](int r) {
            copy_half_kernel<<<cgrid, 256, 0, st>>>(reinterpret_cast<const float4 *>(A[r % NA]), cq, n4);
            return hipGetLastError();
        };
        auto gemm = [&](int r) {
            q3vl::GemmMfArgs g{qf, as, Mt, W[r % NW], S[r % NW], nullptr, nullptr, C, M, N, K};
            return q3vl::launch_gemm_mf(g, false, cus, st);
        };
        float q_hot, q_cold, c_hot, c_cold, g_alone, pair;
        if (time_graph(st, reps, [&](int) { return quant(0); }, &q_hot)) return 1;
        if (time_graph(st, reps, quant, &q_cold)) return 1;
        if (time_graph(st, reps, [&](int) { return copy(0); }, &c_hot)) return 1;
        if (time_graph(st, reps, copy, &c_cold)) return 1;
        CHECK(quant(0));
        if (time_graph(st, reps, gemm, &g_alone)) return 1;
        if (time_graph(st, reps, [&](int r) { hipError_t e = quant(0); return e != hipSuccess ? e : gemm(r); },
                       &pair))
            return 1;
        printf("{\"M\": %d, \"N\": %d, \"K\": %d, \"input_MB\": %.2f, \"quantizer_hot_us\": %.3f, "
               "\"quantizer_cold_us\": %.3f, \"copy_hot_us\": %.3f, \"copy_cold_us\": %.3f, "
               "\"gemm_us\": %.3f, \"quantizer_then_gemm_us\": %.3f, \"quantizer_in_sequence_us\": %.3f}\n",
               M, N, K, na * 4 / 1e6, q_hot, q_cold, c_hot, c_cold, g_alone, pair, pair - g_alone);
        fflush(stdout);
        for (auto p : A) CHECK(hipFree(p));
        for (int c = 0; c < NW; ++c) {
            CHECK(hipFree(W[c]));
            CHECK(hipFree(S[c]));
        }
        CHECK(hipFree(qf));
        CHECK(hipFree(as));
        CHECK(hipFree(C));
        CHECK(hipFree(cq));
    }
    return 0;
}
