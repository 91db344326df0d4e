// linear_timing.cpp -- host-side cost of the engine's linear() drop-in
// (matmul/include/hip_wrapper.hpp) called the way the reference engine calls
// its CPU linear() (matmul/src/cpu_wrapper.cpp:308-396): host activations,
// host weights (uploaded once by the weight registry, then found again by
// address), host output, synchronous.
//
//   linear_timing cfg0 [reps]   config 0's shape, M=1 N=6144 K=2048 (up_proj)
//   linear_timing seq [tokens]  the 197 linears of one decode token of the
//                               Qwen3-VL-2B text decoder in order: per layer
//                               q, k, v, o, gate, up, down, then lm_head
//
// Prints one JSON line: microseconds per call (cfg0) or milliseconds per
// token (seq), median over the timed repetitions, and the same split into the
// pieces linear() does per call, timed separately: pointer-kind queries,
// weight lookup, activation upload, kernel (device-pointer call), result
// download.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../include/hip_wrapper.hpp"
#include "q3vl_int8.h"

namespace {

using clk = std::chrono::steady_clock;
double us_since(clk::time_point t0) {
    return std::chrono::duration<double, std::micro>(clk::now() - t0).count();
}
double median(std::vector<double> v) {
    std::sort(v.begin(), v.end());
    return v[v.size() / 2];
}

// int8 weights in [-127, 127] from a xorshift stream (timing only)
void fill_weights(int8_t *w, size_t n, uint64_t seed) {
    uint64_t x = seed * 0x9E3779B97F4A7C15ull + 1;
    size_t i = 0;
    for (; i + 8 <= n; i += 8) {
        x ^= x << 13, x ^= x >> 7, x ^= x << 17;
        uint64_t v = x;
        for (int b = 0; b < 8; ++b, v >>= 8) w[i + b] = (int8_t)((uint8_t)v == 0x80 ? 0x81 : (uint8_t)v);
    }
    for (; i < n; ++i) w[i] = 1;
}

struct Lin {
    size_t N, K;
    std::vector<int8_t> W;
    std::vector<float> S;
};

Lin make_lin(size_t N, size_t K, uint64_t seed) {
    Lin l{N, K, std::vector<int8_t>(N * K), std::vector<float>(N * (K / 64), 0.01f)};
    fill_weights(l.W.data(), l.W.size(), seed);
    return l;
}

void call(const Lin &l, const float *A, float *C, size_t M) {
    linear(A, l.W.data(), l.S.data(), nullptr, nullptr, C, M, l.N, l.K, true, DType::FP32, DType::INT8,
           DType::FP32, DType::FP32, true, 64);
}

}  // namespace

int main(int argc, char **argv) {
    const char *mode = argc > 1 ? argv[1] : "cfg0";
    if (!strcmp(mode, "cfg0")) {
        const int reps = argc > 2 ? atoi(argv[2]) : 300;
        const size_t M = 1, N = 6144, K = 2048;
        Lin l = make_lin(N, K, 1);
        std::vector<float> A(M * K), C(M * N);
        for (size_t i = 0; i < A.size(); ++i) A[i] = (float)((i * 7919) % 2001) / 1000.0f - 1.0f;
        for (int i = 0; i < 5; ++i) call(l, A.data(), C.data(), M);  // registers the weight
        std::vector<double> t;
        for (int r = 0; r < reps; ++r) {
            const auto t0 = clk::now();
            call(l, A.data(), C.data(), M);
            t.push_back(us_since(t0));
        }
        // the pieces, each timed on its own
        const int8_t *dW = nullptr;
        const float *dS = nullptr;
        if (q3vl_weight_lookup(l.W.data(), l.S.data(), N, K, 64, &dW, &dS) != Q3VL_OK) return 1;
        float *dA = nullptr, *dC = nullptr;
        if (hipMalloc(&dA, M * K * 4) != hipSuccess || hipMalloc(&dC, M * N * 4) != hipSuccess) return 1;
        std::vector<double> tp, tl, tu, tk, td;
        for (int r = 0; r < reps; ++r) {
            hipPointerAttribute_t at{};
            auto t0 = clk::now();
            for (const void *p : {(const void *)A.data(), (const void *)l.W.data(), (const void *)C.data()}) {
                if (hipPointerGetAttributes(&at, p) != hipSuccess) (void)hipGetLastError();
            }
            tp.push_back(us_since(t0));
            t0 = clk::now();
            (void)q3vl_weight_lookup(l.W.data(), l.S.data(), N, K, 64, &dW, &dS);
            tl.push_back(us_since(t0));
            t0 = clk::now();
            (void)hipMemcpy(dA, A.data(), M * K * 4, hipMemcpyHostToDevice);
            tu.push_back(us_since(t0));
            t0 = clk::now();
            (void)q3vl_linear_i8(dA, dW, dS, dC, M, N, K, 64, nullptr, 0, nullptr);
            (void)hipStreamSynchronize(nullptr);
            tk.push_back(us_since(t0));
            t0 = clk::now();
            (void)hipMemcpy(C.data(), dC, M * N * 4, hipMemcpyDeviceToHost);
            td.push_back(us_since(t0));
        }
        printf("{\"mode\": \"cfg0\", \"shape\": [%zu, %zu, %zu], \"reps\": %d, \"us_per_call\": %.2f, "
               "\"pieces_us\": {\"pointer_queries\": %.2f, \"weight_lookup\": %.2f, \"upload_A\": %.2f, "
               "\"kernel_and_sync\": %.2f, \"download_C\": %.2f}}\n",
               M, N, K, reps, median(t), median(tp), median(tl), median(tu), median(tk), median(td));
        (void)hipFree(dA);
        (void)hipFree(dC);
    } else if (!strcmp(mode, "seq")) {
        const int tokens = argc > 2 ? atoi(argv[2]) : 5;
        const size_t H = 2048, I = 6144, QD = 16 * 128, KVD = 8 * 128, V = 151936;
        const int L = 28;
        std::vector<Lin> lins;
        lins.reserve(7 * L + 1);
        uint64_t seed = 10;
        for (int l = 0; l < L; ++l) {
            lins.push_back(make_lin(QD, H, seed++));   // q
            lins.push_back(make_lin(KVD, H, seed++));  // k
            lins.push_back(make_lin(KVD, H, seed++));  // v
            lins.push_back(make_lin(H, QD, seed++));   // o
            lins.push_back(make_lin(I, H, seed++));    // gate
            lins.push_back(make_lin(I, H, seed++));    // up
            lins.push_back(make_lin(H, I, seed++));    // down
        }
        lins.push_back(make_lin(V, H, seed++));  // lm_head
        std::vector<float> x(I, 0.5f), y(V);
        auto token = [&]() {
            for (const Lin &l : lins) call(l, x.data(), y.data(), 1);
        };
        token();  // uploads and registers every weight
        token();
        std::vector<double> t;
        for (int r = 0; r < tokens; ++r) {
            const auto t0 = clk::now();
            token();
            t.push_back(us_since(t0) / 1000.0);
        }
        const double ms = median(t);
        printf("{\"mode\": \"seq\", \"calls_per_token\": %zu, \"tokens\": %d, \"ms_per_token\": %.3f, "
               "\"tok_s\": %.1f, \"us_per_call\": %.2f}\n",
               lins.size(), tokens, ms, 1000.0 / ms, ms * 1000.0 / lins.size());
    } else {
        fprintf(stderr, "usage: %s cfg0|seq [reps]\n", argv[0]);
        return 2;
    }
    q3vl_weight_release_all();
    return 0;
}
