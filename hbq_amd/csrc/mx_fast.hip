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

constexpr int kMxSlots = 12;   // mbit + 6 * fused
constexpr int kMxMaxWords = 10 * 1024 + 2;   // E2M5: binades 2^-7 .. 2^3, plus 2 sentinels
constexpr int kMxMagBytes = 256;             // fp16 magnitudes of up to 128 levels
constexpr int kMxTabBytes = (kMxMagBytes + kMxMaxWords + 15) / 16 * 16;

// per slot: bytes [0, 256) the fp16 magnitude of every level; from byte 256 the
// level of each u: byte 256 + k + 1 for u with fp16 bits lo_bits + k, byte 256
// below the range (level 0), byte 256 + n + 1 at or above it (saturated)
static __device__ __attribute__((aligned(16))) uint8_t g_mx_tab[kMxSlots][kMxTabBytes];
static __device__ int g_mx_status[kMxSlots];
static __device__ int g_mx_bad[kMxSlots];

template <int M>
__device__ __forceinline__ float mx_level_value(int c) {
    const int ef = c >> M, mf = c & ((1 << M) - 1);
    return ef == 0 ? (float)mf * (1.0f / (float)(1 << M)) : (1.0f + (float)mf * (1.0f / (float)(1 << M))) * pow2f(ef - 1);
}

template <int M>
__device__ __forceinline__ uint32_t mx_level(float u, float& mag, bool fused) {
    uint32_t c;
    mag = fabsf(elem_quant<F16, M>(u, c, fused));
    return c & ((1u << (M + 2)) - 1u);
}

template <int M>
__global__ void build_mx_lut_kernel(int slot, int n, uint32_t lo_bits, int fused) {
    const int per = n + 2;
    uint8_t* tab = g_mx_tab[slot];
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < per; i += gridDim.x * blockDim.x) {
        float u, mag;
        if (i == 0) u = 0.f;
        else if (i == per - 1) u = 65504.f;   // fp16 max: saturated
        else u = F16::load((uint16_t)(lo_bits + (uint32_t)(i - 1)));
        const uint32_t lv = mx_level<M>(u, mag, fused);
        tab[kMxMagBytes + i] = (uint8_t)lv;
        // the table stores one magnitude per level: every u of a level must give it
        if (F16::store(mag) != F16::store(mx_level_value<M>((int)lv))) atomicMax(&g_mx_bad[slot], 4);
    }
    const int g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g < (1 << (M + 2))) reinterpret_cast<uint16_t*>(tab)[g] = F16::store(mx_level_value<M>(g));
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        // the constant ends: the largest value below 2^lo has level 0, 2^hi (the
        // first value above the range) is already saturated
        int status = 0;
        float m0, m1, m2;
        if (mx_level<M>(F16::load((uint16_t)(lo_bits - 1u)), m0, fused) != 0u) status = 1;
        if (mx_level<M>(F16::load((uint16_t)(lo_bits + (uint32_t)n)), m1, fused) != (1u << (M + 2)) - 1u) status = 2;
        if (mx_level<M>(65504.f, m2, fused) != (1u << (M + 2)) - 1u || m1 != m2) status = 3;
        g_mx_status[slot] = status;
    }
}

// R16(|lo half of h| * f) into the low half of the result, one v_fma_mix (a single rounding)
__device__ __forceinline__ uint32_t mix_lo(uint32_t h, float f) {
    uint32_t d;
    asm("v_fma_mixlo_f16 %0, |%1|, %2, 0 op_sel_hi:[1,0,0]" : "=v"(d) : "v"(h), "v"(f));
    return d;
}
// R16(|high half of h| * f) into the high half of d
__device__ __forceinline__ void mix_hi(uint32_t& d, uint32_t h, float f) {
    asm("v_fma_mixhi_f16 %0, |%1|, %2, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "+v"(d) : "v"(h), "v"(f));
}

// LPB lanes of 16 elements per block (block 16 or 32), persistent workgroups
template <int M, int LPB>
__global__ __launch_bounds__(kThreads) void mx_fast_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
                                                           uint16_t* __restrict__ scales, uint8_t* __restrict__ codes,
                                                           int64_t nb, int slot, int n, uint32_t lo_m1, MxParams p) {
    constexpr int block = kV * LPB;
    constexpr int blocks_per_wg = kThreads / LPB;
    extern __shared__ __attribute__((aligned(16))) uint8_t tab[];
    {   // copy the table in 16-byte pieces
        const uint4* src = reinterpret_cast<const uint4*>(g_mx_tab[slot]);
        uint4* dst = reinterpret_cast<uint4*>(tab);
        for (int i = threadIdx.x; i < (kMxMagBytes + n + 2 + 15) / 16; i += kThreads) dst[i] = src[i];
    }
    // the fp16 log2 thresholds of the shared scale, after the table
    float* l2t = reinterpret_cast<float*>(tab + (kMxMagBytes + n + 2 + 15) / 16 * 16);
    for (int i = threadIdx.x; i < 80; i += kThreads) l2t[i] = i < 40 ? kLog2FloorF16[i] : kLog2RoundF16[i - 40];
    __syncthreads();
    const LdsLog2 lt{l2t, l2t + 40};
    const uint16_t* mags = reinterpret_cast<const uint16_t*>(tab);
    const uint8_t* lvls = tab + kMxMagBytes;   // lvls[k + 1] for u with fp16 bits lo_bits + k

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
        const float s = mx_shared_scale<F16>(amax, p, lt);
        const float rs = 1.0f / s;

        uint32_t y2[8];
        uint32_t cout[kV];
        if (__builtin_expect((m2 > 0x7c00u) | !(s > 0.f && s < __builtin_inff()), 0)) {
            // a NaN in the block, or a scale that rounds to 0 or inf in fp16 (an 8-bit
            // scale exponent): the generic element path
            float out[kV];
#pragma unroll
            for (int i = 0; i < kV; ++i) {
                const float v = F16::load((uint16_t)(i & 1 ? w[i / 2] >> 16 : w[i / 2] & 0xffffu));
                const float yv = p.pot ? F16::round(v * rs) : div_T<F16>(v, s, rs);
                const float q = elem_quant<F16, M>(yv, cout[i], p.fused);
                out[i] = F16::round(q * s);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i)
                y2[i] = (uint32_t)F16::store(out[2 * i]) | ((uint32_t)F16::store(out[2 * i + 1]) << 16);
        } else {
            // u = R16(|x| / s) of each element, packed in pairs like x: for a power-of-two
            // scale the product is exact; for an FP scale R16(|x| * R32(1/s)) (one
            // rounding) equals R16(|x| / s) unless the quotient is below 2^-14
            uint32_t u2[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                u2[i] = mix_lo(w[i], rs);
                mix_hi(u2[i], w[i], rs);
            }
            if (!p.pot) {
                u16x2_t mn = __builtin_bit_cast(u16x2_t, u2[0]);
#pragma unroll
                for (int i = 1; i < 8; ++i) mn = __builtin_elementwise_min(mn, __builtin_bit_cast(u16x2_t, u2[i]));
                if ((mn.x <= 0x0400u) | (mn.y <= 0x0400u)) {   // near or in the subnormal range: divide
#pragma unroll
                    for (int i = 0; i < kV; ++i) {
                        const uint32_t key = i & 1 ? u2[i / 2] >> 16 : u2[i / 2] & 0xffffu;
                        if (key <= 0x0400u) {
                            const float a = fabsf(F16::load((uint16_t)(i & 1 ? w[i / 2] >> 16 : w[i / 2] & 0xffffu)));
                            const uint32_t k2 = F16::store(a / s);
                            u2[i / 2] = i & 1 ? (u2[i / 2] & 0xffffu) | (k2 << 16) : (u2[i / 2] & 0xffff0000u) | k2;
                        }
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                uint32_t lv[2];
                u16x2_t q2;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int key = (int)(h ? u2[i] >> 16 : u2[i] & 0xffffu);
                    int k;   // word index k + 1 clamped to [0, n + 1] in one v_med3_i32
                    asm("v_med3_i32 %0, %1, 0, %2" : "=v"(k) : "v"(key - (int)lo_m1), "s"(n + 1));
                    lv[h] = lvls[k];
                    q2[h] = mags[lv[h]];
                }
                uint32_t o2 = mix_lo(__builtin_bit_cast(uint32_t, q2), s);   // R16(q * s): exact product
                mix_hi(o2, __builtin_bit_cast(uint32_t, q2), s);
                // the sign of x unless u is +-0 (the reference's u == 0 gives +0 and code 0):
                // bit 15 of each half of u2 + 0x7fff7fff is set iff that half is nonzero
                // (u <= 0x7c00, so no carry crosses the halves)
                const uint32_t sg = w[i] & (u2[i] + 0x7fff7fffu) & 0x80008000u;
                y2[i] = o2 | sg;
                cout[2 * i] = lv[0] | (((sg >> 15) & 1u) << (M + 2));
                cout[2 * i + 1] = lv[1] | ((sg >> 31) << (M + 2));
            }
        }
        if (valid) {
            u32x4_t* yq = reinterpret_cast<u32x4_t*>(y + off);
            __builtin_nontemporal_store((u32x4_t){y2[0], y2[1], y2[2], y2[3]}, yq);
            __builtin_nontemporal_store((u32x4_t){y2[4], y2[5], y2[6], y2[7]}, yq + 1);
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
int build_mx_slot(int slot, int n, uint32_t lo_bits, int fused, hipStream_t st) {
    hipLaunchKernelGGL((build_mx_lut_kernel<M>), dim3(32), dim3(256), 0, st, slot, n, lo_bits, fused);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return -hbq_fail(HBQ_ERR_HIP, "MX level table build failed: %s", hipGetErrorString(e));
    int status = -1, bad = -1;
    e = hipMemcpyFromSymbol(&status, HIP_SYMBOL(g_mx_status), sizeof(int), sizeof(int) * slot,
                            hipMemcpyDeviceToHost);
    if (e == hipSuccess)
        e = hipMemcpyFromSymbol(&bad, HIP_SYMBOL(g_mx_bad), sizeof(int), sizeof(int) * slot, hipMemcpyDeviceToHost);
    if (e != hipSuccess)
        return -hbq_fail(HBQ_ERR_HIP, "MX level table status read failed: %s", hipGetErrorString(e));
    return status > bad ? status : bad;
}

template <int M, int LPB>
int launch_mx_fast(const void* x, void* y, void* scales, void* codes, int64_t nb, int slot, int n, uint32_t lo_bits,
                   const MxParams& p, int dev, hipStream_t st) {
    const size_t lds = (size_t)((kMxMagBytes + n + 2 + 15) / 16) * 16 + 80 * sizeof(float);
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
                       (uint16_t*)scales, (uint8_t*)codes, nb, slot, n, lo_bits - 1u, p);
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
    const int slot = mbit + 6 * (p.fused != 0);   // one table per element format and rounding
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
            const int fz = p.fused != 0;
            const int rc = mbit == 1 ? build_mx_slot<1>(slot, n, lo_bits, fz, st)
                           : mbit == 2 ? build_mx_slot<2>(slot, n, lo_bits, fz, st)
                           : mbit == 3 ? build_mx_slot<3>(slot, n, lo_bits, fz, st)
                                       : build_mx_slot<5>(slot, n, lo_bits, fz, st);
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
