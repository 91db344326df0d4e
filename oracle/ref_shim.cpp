// ref_shim.cpp -- C entry points over the reference's own sources, compiled
// from /root/reference by oracle/Makefile into oracle/_ref/ (never committed).
//
// TEST INFRASTRUCTURE ONLY. It lets tests and the golden-vector writer call the
// reference's real linear() (matmul/src/cpu_wrapper.cpp:308) and swiglu()
// (layers/src/text_layer.cpp:420), and lets bench.py time the reference CPU
// path. Nothing here is linked into the HIP library.
#include <cstddef>
#include <cstdint>
#include <vector>

#include "matmul/module.hpp"
#include "layers/include/text_layer.hpp"

namespace {
// Tensor's destructor unmaps buffers it does not own (utils/src/tensor.cpp:
// 83-101), so wrappers over caller memory must drop their pointers first.
struct Wrap {
    Tensor t;
    Wrap(std::vector<size_t> shape, void *buf) : t(shape, buf, DType::FP32) {}
    ~Wrap() { t.buf = nullptr; t.scale_buf = nullptr; }
};
}  // namespace

extern "C" {

// The int8 group-quantized branch of linear(): FP32 A, INT8 B [N,K]
// (mat_B_transpose=true), FP32 group scales, FP32 C, no bias.
void ref_linear_i8(const float *A, const int8_t *W, const float *S, float *C,
                   size_t M, size_t N, size_t K, size_t gs) {
    linear(A, W, S, nullptr, nullptr, C, M, N, K, true, DType::FP32,
           DType::INT8, DType::FP32, DType::FP32, true, gs);
}

void ref_swiglu(float *gate, const float *up, size_t n) {
    Wrap g({n}, gate);
    Wrap u({n}, const_cast<float *>(up));
    swiglu(&g.t, &u.t, n);
}

}  // extern "C"
