// matmul/module.hpp -- drop-in replacement of the engine's matmul module
// (matmul/module.hpp:1-2 of the reference), backed by libq3vl_int8.so.
#pragma once

#include "include/hip_wrapper.hpp"
