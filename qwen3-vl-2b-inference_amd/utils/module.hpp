// utils/module.hpp -- stand-in for the engine's utils module when this
// package is built on its own. It defines only what the matmul drop-in needs,
// with the engine's ABI: DType::Type values FP32=0, INT32=1, FP16=2, INT8=3,
// INT4=4 (utils/include/tensor.hpp:38 of the reference engine). Inside the
// engine, matmul/ includes the engine's own ../../utils/module.hpp instead.
#pragma once

#include <cstddef>
#include <cstdint>

struct DType {
    enum Type { FP32, INT32, FP16, INT8, INT4 };
};

struct PtrPair {
    const void *buf;
    const void *scale;
};
