// Elementwise pieces of the Llama decoder around the quantized linears, fused
// with torch's bits: the RMSNorm of the residual stream (with the residual add
// that precedes it) and the SiLU-gated product of the MLP.  Every step is what
// torch's eager kernels compute: each op in fp32 on the T values (Python
// scalars as fp32), rounded to T once per op, with torch's float -> bf16 NaN
// (0x7FC0).  8 elements (16 bytes) a thread.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <initializer_list>

#include "hbq_capi_internal.h"
#include "model_math.h"
#include "quant_common.h"

namespace hbq {
namespace {

template <class T>
__device__ __forceinline__ void unpack8(const u32x4& v, float (&x)[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = T::load((uint16_t)(w[e / 2] >> (16 * (e % 2))));
}

template <class T>
__device__ __forceinline__ u32x4 pack8(const float (&y)[8]) {
    uint32_t w[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) w[p] = store_t<T>(y[2 * p]) | (store_t<T>(y[2 * p + 1]) << 16);
    return (u32x4){w[0], w[1], w[2], w[3]};
}

// s = R(x + res) (when res is given, written to sum), sq = s * s in fp32
// (h.float().pow(2) of the RMSNorm: the square of a 16-bit value is exact in fp32)
template <class T>
__global__ __launch_bounds__(kThreads) void rms_prep_kernel(const uint16_t* x, const uint16_t* __restrict__ res,
                                                            uint16_t* sum, float* __restrict__ sq,
                                                            int64_t n8) {
    const int64_t u = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (u >= n8) return;
    float s[8];
    unpack8<T>(*reinterpret_cast<const u32x4*>(x + 8 * u), s);
    if (res) {
        float r[8];
        unpack8<T>(*reinterpret_cast<const u32x4*>(res + 8 * u), r);
#pragma unroll
        for (int e = 0; e < 8; ++e) s[e] = s[e] + r[e];
        const u32x4 o = pack8<T>(s);
        *reinterpret_cast<u32x4*>(sum + 8 * u) = o;
        unpack8<T>(o, s);
    }
    float4* q = reinterpret_cast<float4*>(sq + 8 * u);
    q[0] = make_float4(s[0] * s[0], s[1] * s[1], s[2] * s[2], s[3] * s[3]);
    q[1] = make_float4(s[4] * s[4], s[5] * s[5], s[6] * s[6], s[7] * s[7]);
}

// y = R(w * R(R32(x * r[row]))) (cols % 8 == 0); r = rsqrt(var + eps) comes from
// torch, whose rsqrt can differ from this build's rsqrtf in the last bit
template <class T>
__global__ __launch_bounds__(kThreads) void rms_apply_kernel(const uint16_t* __restrict__ x,
                                                             const float* __restrict__ rs,
                                                             const uint16_t* __restrict__ w, uint16_t* __restrict__ y,
                                                             int64_t n8, int64_t cols8) {
    const int64_t u = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (u >= n8) return;
    const int64_t row = u / cols8, c8 = u - row * cols8;
    const float r = rs[row];
    float xv[8], wv[8], o[8];
    unpack8<T>(*reinterpret_cast<const u32x4*>(x + 8 * u), xv);
    unpack8<T>(*reinterpret_cast<const u32x4*>(w + 8 * c8), wv);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = rms_apply_one<T>(xv[e], r, wv[e]);
    *reinterpret_cast<u32x4*>(y + 8 * u) = pack8<T>(o);
}

// y = R(R(g / (1 + exp(-g))) * u): torch's silu (fp32 division by 1 + expf(-g)) and product
template <class T>
__global__ __launch_bounds__(kThreads) void silu_mul_kernel(const uint16_t* __restrict__ g,
                                                            const uint16_t* __restrict__ up,
                                                            uint16_t* __restrict__ y, int64_t n8) {
    const int64_t u = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (u >= n8) return;
    float gv[8], uv[8], o[8];
    unpack8<T>(*reinterpret_cast<const u32x4*>(g + 8 * u), gv);
    unpack8<T>(*reinterpret_cast<const u32x4*>(up + 8 * u), uv);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = silu_mul_one<T>(gv[e], uv[e]);
    *reinterpret_cast<u32x4*>(y + 8 * u) = pack8<T>(o);
}

int check_common(int dtype, int64_t n, std::initializer_list<const void*> ptrs) {
    if (dtype != kF16 && dtype != kBF16) return hbq_fail(HBQ_ERR_UNSUPPORTED, "fp16 or bf16 tensors only");
    if (n < 0) return hbq_fail(HBQ_ERR_INVALID, "negative size");
    if (n % 8) return hbq_fail(HBQ_ERR_UNSUPPORTED, "the element count must be a multiple of 8");
    for (const void* p : ptrs)
        if (p && (uintptr_t)p % 16) return hbq_fail(HBQ_ERR_INVALID, "tensors must be 16-byte aligned");
    if ((n / 8 + kThreads - 1) / kThreads > 0x7fffffff) return hbq_fail(HBQ_ERR_INVALID, "tensor too large");
    return 0;
}

}  // namespace
}  // namespace hbq

using namespace hbq;

extern "C" {

int hbq_rms_prep(const void* x, const void* res, void* sum, float* sq, int64_t n, int dtype, void* stream) {
    hbq_clear_error();
    if (int rc = check_common(dtype, n, {x, res, sum, sq})) return rc;
    if (n == 0) return 0;
    if (!x || !sq || (res && !sum)) return hbq_fail(HBQ_ERR_INVALID, "null pointer");
    const int64_t n8 = n / 8;
    const dim3 grid((unsigned)((n8 + kThreads - 1) / kThreads));
    if (dtype == kF16)
        hipLaunchKernelGGL(rms_prep_kernel<F16>, grid, dim3(kThreads), 0, (hipStream_t)stream, (const uint16_t*)x,
                           (const uint16_t*)res, (uint16_t*)sum, sq, n8);
    else
        hipLaunchKernelGGL(rms_prep_kernel<BF16>, grid, dim3(kThreads), 0, (hipStream_t)stream, (const uint16_t*)x,
                           (const uint16_t*)res, (uint16_t*)sum, sq, n8);
    return hbq_check_launch("hbq_rms_prep");
}

int hbq_rms_apply(const void* x, const float* rs, const void* w, void* y, int64_t rows, int64_t cols, int dtype,
                  void* stream) {
    hbq_clear_error();
    if (rows < 0 || cols < 0) return hbq_fail(HBQ_ERR_INVALID, "negative size");
    if (cols % 8) return hbq_fail(HBQ_ERR_UNSUPPORTED, "the row length must be a multiple of 8");
    if (int rc = check_common(dtype, rows * cols, {x, w, y})) return rc;
    if (rows == 0 || cols == 0) return 0;
    if (!x || !rs || !w || !y) return hbq_fail(HBQ_ERR_INVALID, "null pointer");
    const int64_t n8 = rows * cols / 8;
    const dim3 grid((unsigned)((n8 + kThreads - 1) / kThreads));
    if (dtype == kF16)
        hipLaunchKernelGGL(rms_apply_kernel<F16>, grid, dim3(kThreads), 0, (hipStream_t)stream, (const uint16_t*)x,
                           rs, (const uint16_t*)w, (uint16_t*)y, n8, cols / 8);
    else
        hipLaunchKernelGGL(rms_apply_kernel<BF16>, grid, dim3(kThreads), 0, (hipStream_t)stream, (const uint16_t*)x,
                           rs, (const uint16_t*)w, (uint16_t*)y, n8, cols / 8);
    return hbq_check_launch("hbq_rms_apply");
}

int hbq_silu_mul(const void* g, const void* u, void* y, int64_t n, int dtype, void* stream) {
    hbq_clear_error();
    if (int rc = check_common(dtype, n, {g, u, y})) return rc;
    if (n == 0) return 0;
    if (!g || !u || !y) return hbq_fail(HBQ_ERR_INVALID, "null pointer");
    const int64_t n8 = n / 8;
    const dim3 grid((unsigned)((n8 + kThreads - 1) / kThreads));
    if (dtype == kF16)
        hipLaunchKernelGGL(silu_mul_kernel<F16>, grid, dim3(kThreads), 0, (hipStream_t)stream, (const uint16_t*)g,
                           (const uint16_t*)u, (uint16_t*)y, n8);
    else
        hipLaunchKernelGGL(silu_mul_kernel<BF16>, grid, dim3(kThreads), 0, (hipStream_t)stream, (const uint16_t*)g,
                           (const uint16_t*)u, (uint16_t*)y, n8);
    return hbq_check_launch("hbq_silu_mul");
}

}  // extern "C"
