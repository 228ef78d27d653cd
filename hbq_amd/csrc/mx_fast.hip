// Table-driven MXFP / NVFP quantize-dequantize for fp16 inputs
// (MXFPQuantizer.get_shared_scale + q, src/quantizer.py:481-539).
//
// After the shared scale, the element path of the reference is
//   u = R16(x / s),  q = lpfp(u),  y = R16(q * s)
// and lpfp (make_fp_quant, src/quantizer.py:187-257) is a function of the
// 16-bit value u alone.  So one table indexed by the bits of |u| gives the
// element level (the magnitude code) and the level's magnitude as fp16, for
// the binades [2^-(m+2), 2^3) where the level is not constant; below it every
// u quantizes to level 0, at or above 8 every u saturates.  The table is
// built on the GPU by the same device element quantizer as the generic kernel
// (so it agrees with it by construction), its constant ends are checked, and
// each persistent workgroup copies it into LDS.  Per element what remains is
// R16(|x| * 1/s) (exact for a power-of-two scale; for the E5M3 scale of NVFP
// it equals R16(|x| / s) outside the fp16 subnormal range, and the kernel
// divides where a quotient falls there), one LDS read, R16(q * s) and the
// sign: the output and the code take the sign of x unless u is +-0, where the
// reference gives +0 and code 0 (src/quantizer.py:241-245).  A block holding
// a NaN, or whose scale is 0 or inf in fp16, takes the generic element path.
#include <hip/hip_runtime.h>
#include <math.h>
#include <mutex>
#include <stdint.h>

#include "hbq_capi_internal.h"
#include "mx_fast.h"
#include "quant_common.h"

namespace hbq {

constexpr int kMxSlots = 8;
constexpr int kMxMaxEntries = 10 * 1024 + 2;   // E2M5: binades 2^-7 .. 2^3

// per slot: word k + 1 describes u with fp16 bits lo_bits + k; word 0 is below
// the range (level 0, magnitude 0), word n + 1 at or above it (saturated).
// Word layout: bits 0-7 the level, bits 16-31 the fp16 bits of its magnitude.
static __device__ uint32_t g_mx_lut[kMxSlots][kMxMaxEntries];
static __device__ int g_mx_status[kMxSlots];

template <int M>
__device__ __forceinline__ uint32_t mx_word(float u) {
    uint32_t c;
    const float q = elem_quant<F16, M>(u, c);
    return (c & ((1u << (M + 2)) - 1u)) | ((uint32_t)F16::store(fabsf(q)) << 16);
}

template <int M>
__global__ void build_mx_lut_kernel(int slot, int n, uint32_t lo_bits) {
    const int per = n + 2;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < per; i += gridDim.x * blockDim.x) {
        float u;
        if (i == 0) u = 0.f;
        else if (i == per - 1) u = 65504.f;   // fp16 max: saturated
        else u = F16::load((uint16_t)(lo_bits + (uint32_t)(i - 1)));
        g_mx_lut[slot][i] = mx_word<M>(u);
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        // the constant ends: the largest value below 2^lo has level 0, 2^hi (the
        // first value above the range) is already saturated
        int status = 0;
        if ((mx_word<M>(F16::load((uint16_t)(lo_bits - 1u))) & 0xffu) != 0u) status = 1;
        if (mx_word<M>(F16::load((uint16_t)(lo_bits + (uint32_t)n))) != mx_word<M>(65504.f)) status = 2;
        if ((mx_word<M>(65504.f) & 0xffu) != (1u << (M + 2)) - 1u) status = 3;
        g_mx_status[slot] = status;
    }
}

// LPB lanes of 16 elements per block (block 16 or 32), persistent workgroups
template <int M, int LPB>
__global__ __launch_bounds__(kThreads) void mx_fast_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
                                                           uint16_t* __restrict__ scales, uint8_t* __restrict__ codes,
                                                           int64_t nb, int slot, int n, uint32_t lo_bits, MxParams p) {
    constexpr int block = kV * LPB;
    constexpr int blocks_per_wg = kThreads / LPB;
    extern __shared__ uint32_t lut[];
    for (int i = threadIdx.x; i < n + 2; i += kThreads) lut[i] = g_mx_lut[slot][i];
    __syncthreads();

    const int li = (int)(threadIdx.x & (LPB - 1));
    const int64_t ntiles = (nb + blocks_per_wg - 1) / blocks_per_wg;
    typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
    typedef uint16_t u16x2_t __attribute__((ext_vector_type(2)));

    for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const int64_t gb = tile * blocks_per_wg + (threadIdx.x / LPB);
        const bool valid = gb < nb;
        const int64_t off = (valid ? gb : 0) * (int64_t)block + (int64_t)li * kV;
        uint32_t w[8];
        if (valid) {
            const u32x4_t* q = reinterpret_cast<const u32x4_t*>(x + off);
            const u32x4_t a = __builtin_nontemporal_load(q), b = __builtin_nontemporal_load(q + 1);
            w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w; w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) w[i] = 0u;
        }
        // block max of |x| over the 16-bit patterns (NaN patterns sort above inf)
        u16x2_t mp = __builtin_bit_cast(u16x2_t, w[0] & 0x7fff7fffu);
#pragma unroll
        for (int i = 1; i < 8; ++i) mp = __builtin_elementwise_max(mp, __builtin_bit_cast(u16x2_t, w[i] & 0x7fff7fffu));
        uint32_t m2 = mp.x > mp.y ? (uint32_t)mp.x : (uint32_t)mp.y;
        if constexpr (LPB == 2) {
            const uint32_t o = (uint32_t)__builtin_amdgcn_mov_dpp((int)m2, 0xB1, 0xf, 0xf, true);   // quad_perm [1,0,3,2]
            m2 = m2 > o ? m2 : o;
        }
        const float amax = F16::load((uint16_t)m2);
        const float s = mx_shared_scale<F16>(amax, p);
        const float rs = 1.0f / s;

        float out[kV];
        uint32_t cout[kV];
        if (__builtin_expect((m2 > 0x7c00u) | !(s > 0.f && s < __builtin_inff()), 0)) {
            // a NaN in the block, or a scale that rounds to 0 or inf in fp16 (an 8-bit
            // scale exponent): the generic element path
#pragma unroll
            for (int i = 0; i < kV; ++i) {
                const float v = F16::load((uint16_t)(i & 1 ? w[i / 2] >> 16 : w[i / 2] & 0xffffu));
                const float yv = p.pot ? F16::round(v * rs) : div_T<F16>(v, s, rs);
                const float q = elem_quant<F16, M>(yv, cout[i]);
                out[i] = F16::round(q * s);
            }
        } else {
            uint32_t key[kV];
            float pmin = 65504.f;
#pragma unroll
            for (int i = 0; i < kV; ++i) {
                const float a = fabsf(F16::load((uint16_t)(i & 1 ? w[i / 2] >> 16 : w[i / 2] & 0xffffu)));
                const float pr = a * rs;
                pmin = fminf(pmin, pr);
                key[i] = F16::store(pr);   // R16(|x| * 1/s)
            }
            if (!p.pot && pmin < 6.103515625e-05f) {   // fp16 subnormal quotients can be exact ties: divide
#pragma unroll
                for (int i = 0; i < kV; ++i) {
                    const float a = fabsf(F16::load((uint16_t)(i & 1 ? w[i / 2] >> 16 : w[i / 2] & 0xffffu)));
                    if (a * rs < 6.103515625e-05f) key[i] = F16::store(a / s);
                }
            }
#pragma unroll
            for (int i = 0; i < kV; ++i) {
                int k;   // clamp to [-1, n]; word k + 1
                asm("v_med3_i32 %0, %1, -1, %2" : "=v"(k) : "v"((int)key[i] - (int)lo_bits), "s"(n));
                const uint32_t e = lut[k + 1];
                const uint32_t xs = (i & 1 ? w[i / 2] >> 31 : (w[i / 2] >> 15) & 1u) & (key[i] != 0u ? 1u : 0u);
                const float o = F16::round(F16::load((uint16_t)(e >> 16)) * s);
                out[i] = xs ? -o : o;
                cout[i] = (e & 0xffu) | (xs << (M + 2));
            }
        }
        if (valid) {
            store16<F16>(y + off, out);
            if (codes) {
                if constexpr (M == 1) {
                    uint32_t w0 = 0, w1 = 0;
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        w0 |= (cout[i] & 0xfu) << (4 * i);
                        w1 |= (cout[8 + i] & 0xfu) << (4 * i);
                    }
                    *reinterpret_cast<uint2*>(codes + off / 2) = make_uint2(w0, w1);
                } else {
                    uint32_t cw[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        cw[i] = (cout[4 * i] & 0xffu) | ((cout[4 * i + 1] & 0xffu) << 8) |
                                ((cout[4 * i + 2] & 0xffu) << 16) | ((cout[4 * i + 3] & 0xffu) << 24);
                    *reinterpret_cast<uint4*>(codes + off) = make_uint4(cw[0], cw[1], cw[2], cw[3]);
                }
            }
            if (scales != nullptr && li == 0) scales[gb] = F16::store(s);
        }
    }
}

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mx_mu;
int g_mx_mbit[kMaxDevices][kMxSlots];   // element mantissa bits of the slot's table, 0: empty
int g_mx_cus[kMaxDevices];

template <int M>
int build_mx_slot(int slot, int n, uint32_t lo_bits, hipStream_t st) {
    hipLaunchKernelGGL((build_mx_lut_kernel<M>), dim3(32), dim3(256), 0, st, slot, n, lo_bits);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return -hbq_fail(HBQ_ERR_HIP, "MX level table build failed: %s", hipGetErrorString(e));
    int status = -1;
    e = hipMemcpyFromSymbol(&status, HIP_SYMBOL(g_mx_status), sizeof(int), sizeof(int) * slot,
                            hipMemcpyDeviceToHost);
    if (e != hipSuccess)
        return -hbq_fail(HBQ_ERR_HIP, "MX level table status read failed: %s", hipGetErrorString(e));
    return status;
}

template <int M, int LPB>
int launch_mx_fast(const void* x, void* y, void* scales, void* codes, int64_t nb, int slot, int n, uint32_t lo_bits,
                   const MxParams& p, int dev, hipStream_t st) {
    const size_t lds = (size_t)(n + 2) * 4;
    auto kern = mx_fast_kernel<M, LPB>;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kThreads, lds) != hipSuccess || per_cu <= 0)
        return 0;
    const int64_t blocks_per_wg = kThreads / LPB;
    const int64_t ntiles = (nb + blocks_per_wg - 1) / blocks_per_wg;
    const int64_t resident = (int64_t)g_mx_cus[dev] * per_cu;
    const int64_t rounds = (ntiles + resident - 1) / resident;
    const int64_t grid = (ntiles + rounds - 1) / rounds;
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(kThreads), lds, st, (const uint16_t*)x, (uint16_t*)y,
                       (uint16_t*)scales, (uint8_t*)codes, nb, slot, n, lo_bits, p);
    return 1;
}

template <int M>
int mx_fast_block(int block, const void* x, void* y, void* scales, void* codes, int64_t nb, int slot, int n,
                  uint32_t lo_bits, const MxParams& p, int dev, hipStream_t st) {
    if (block == 16) return launch_mx_fast<M, 1>(x, y, scales, codes, nb, slot, n, lo_bits, p, dev, st);
    return launch_mx_fast<M, 2>(x, y, scales, codes, nb, slot, n, lo_bits, p, dev, st);
}

}  // namespace
}  // namespace hbq

using namespace hbq;

int hbq_mx_fast_try(const void* x, void* y, void* scales, void* codes, int64_t rows, int64_t cols, int dtype,
                    int block, int mbit, const MxParams& p, hipStream_t st) {
    if (dtype != kF16 || p.per_tensor) return 0;
    if (mbit != 1 && mbit != 2 && mbit != 3 && mbit != 5) return 0;
    if ((block != 16 && block != 32) || cols % block) return 0;
    if (((uintptr_t)x % 16) || ((uintptr_t)y % 16) || (codes && ((uintptr_t)codes % 16))) return 0;
    const int lo = -(mbit + 2), hi = 3;   // table range [2^lo, 2^hi)
    const int n = (hi - lo) << 10;
    const uint32_t lo_bits = (uint32_t)(15 + lo) << 10;

    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
    const int slot = mbit;   // one table per element format
    {
        std::lock_guard<std::mutex> g(g_mx_mu);
        if (g_mx_cus[dev] == 0) {
            int cus = 0;
            if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
                return 0;
            g_mx_cus[dev] = cus;
        }
        if (g_mx_mbit[dev][slot] < 0) return 0;
        if (g_mx_mbit[dev][slot] == 0) {
            const int rc = mbit == 1 ? build_mx_slot<1>(slot, n, lo_bits, st)
                           : mbit == 2 ? build_mx_slot<2>(slot, n, lo_bits, st)
                           : mbit == 3 ? build_mx_slot<3>(slot, n, lo_bits, st)
                                       : build_mx_slot<5>(slot, n, lo_bits, st);
            if (rc < 0) return rc;
            g_mx_mbit[dev][slot] = rc == 0 ? mbit : -1;
            if (rc != 0) return 0;
        }
    }
    const int64_t nb = rows * (cols / block);
    if (nb == 0) return 1;
    switch (mbit) {
        case 1: return mx_fast_block<1>(block, x, y, scales, codes, nb, slot, n, lo_bits, p, dev, st);
        case 2: return mx_fast_block<2>(block, x, y, scales, codes, nb, slot, n, lo_bits, p, dev, st);
        case 3: return mx_fast_block<3>(block, x, y, scales, codes, nb, slot, n, lo_bits, p, dev, st);
        default: return mx_fast_block<5>(block, x, y, scales, codes, nb, slot, n, lo_bits, p, dev, st);
    }
}
