// Per-element math of the decoder passes around the quantized linears, shared by
// their own kernels (model_ops.hip) and by the activation quantizer that can take
// their output as its input without a round trip through memory (hbq_fast.hip).
// Each step is what torch's eager kernels compute: fp32 on the T values, rounded
// to T once per op; torch's float -> bf16 conversion gives 0x7FC0 for every NaN.
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "hbq_numeric.h"

namespace hbq {

template <class T>
__device__ __forceinline__ uint32_t store_t(float v) {
    return (T::dt == kBF16 && v != v) ? 0x7FC0u : (uint32_t)T::store(v);
}

// RMSNorm, second half: R(w * R(R32(x * r))) with r = rsqrt(var + eps) of the row
// (the `h * rs`, `.to(dtype)` and `weight *` steps of LlamaRMSNorm)
template <class T>
__device__ __forceinline__ float rms_apply_one(float x, float r, float w) {
    float h = x * r;
    asm("" : "+v"(h));               // the fp32 product is rounded before the conversion
    return w * T::round(h);
}

// R(R(g / (1 + exp(-g))) * u): torch's silu (fp32 division by 1 + expf(-g)) and product
template <class T>
__device__ __forceinline__ float silu_mul_one(float g, float u) {
    float d = 1.0f + expf(-g);
    asm("" : "+v"(d));
    const float s = g / d;
    return T::round(s) * u;
}

}  // namespace hbq
