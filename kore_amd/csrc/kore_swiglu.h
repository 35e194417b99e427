// kore_swiglu.h - kore's SwiGLU of one value, shared by the row-wise kernels
// and the batched matmul's gate/up fix-up.  Internal to libkore_qmv.so.
#pragma once

#include <hip/hip_runtime.h>

namespace kore_qmv_gpu {

// kore's SwiGLU of one value (kore.cpp:1466-1467): g / (1.0f + std::exp(-g)) * u.
// exp is taken in double and rounded to float (glibc's expf agrees with that
// correctly rounded value except in rare hard cases); the division is rounded
// once from double like kore's float division.
__device__ __forceinline__ float kore_swiglu(float g, float u) {
    const float ex = (float)exp(-(double)g);
    const float den = 1.0f + ex;
    const float q = (float)((double)g / (double)den);
    return q * u;
}

}  // namespace kore_qmv_gpu
