// Table-driven MXFP / NVFP quantize-dequantize for fp16 inputs
// (MXFPQuantizer.get_shared_scale + q, src/quantizer.py:481-539).
//
// After the shared scale, the element path of the reference is
//   u = R16(x / s),  q = lpfp(u),  y = R16(q * s)
// and lpfp (make_fp_quant, src/quantizer.py:187-257) is a function of the
// 16-bit value u alone.  So one byte table indexed by the bits of |u| gives, in one
// LDS read, the element level (the magnitude code) for the binades [2^-(m+2), 2^3)
// where the level is not constant; below it every u quantizes to level 0, at or
// above 8 every u saturates.  The level's value follows from its code in three
// packed fp16 instructions for two elements (see the kernel), which keeps the
// table a quarter of the size of one that also held the value: each workgroup's
// copy of it into LDS costs that much less (MXFP8 13%, MXFP4 3-4% faster).  The table is built on the GPU by the same device
// element quantizer as the generic kernel (so it agrees with it by
// construction), its constant ends are checked, and each persistent workgroup
// copies it into LDS.  Per element what remains is R16(|x| * 1/s) (exact for a
// power-of-two scale; for the E5M3 scale of NVFP it equals R16(|x| / s)
// outside the fp16 subnormal range, and the kernel divides where a quotient
// falls there), the LDS read, R16(q * s) and the sign: the output and the code
// take the sign of x unless u is +-0, where the reference gives +0 and code 0
// (src/quantizer.py:241-245).  A wave tile holding a NaN, or a block whose
// scale is 0 or inf in fp16, takes the generic element path.
//
// Lane mapping: a wave works on 1024 consecutive elements, lane l holding
// elements [8 l, 8 l + 8) and [512 + 8 l, 512 + 8 l + 8), so that each of the
// wave's global load and store instructions covers one contiguous range (1 KB
// of x or y, 256 / 512 B of codes).  A block (16 or 32 elements) is 2 or 4
// neighbouring lanes of one half.  A traffic-only kernel streaming y + codes +
// scales this way measured 6.4 TB/s against 5.1 TB/s with 16 contiguous elements
// per lane.  Plain (not nontemporal) loads and stores measured slightly faster here.
#include <hip/hip_runtime.h>
#include <math.h>
#include <mutex>
#include <stdint.h>

#include "hbq_capi_internal.h"
#include "mx_fast.h"
#include "quant_common.h"

namespace hbq {

constexpr int kMxSlots = 12;   // mbit + 6 * fused
// E2M5: binades 2^-7 .. 2^3 plus 2 sentinels (bytes), rounded up so that every row starts
// 16-byte aligned; the kernel copies (n + 2) bytes in 16-byte pieces
constexpr int kMxMaxWords = 10 * 1024 + 8;
constexpr int kMxThreads = 512;              // 8 waves share one LDS copy of the table

// per slot, as bytes: byte k + 1 is the level of u with fp16 bits lo_bits + k, byte 0
// below the range (level 0), byte n + 1 at or above it (saturated)
static __device__ __attribute__((aligned(16))) uint32_t g_mx_tab[kMxSlots][kMxMaxWords];
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
    uint32_t* tab = g_mx_tab[slot];
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < per; i += gridDim.x * blockDim.x) {
        float u, mag;
        if (i == 0) u = 0.f;
        else if (i == per - 1) u = 65504.f;   // fp16 max: saturated
        else u = F16::load((uint16_t)(lo_bits + (uint32_t)(i - 1)));
        const uint32_t lv = mx_level<M>(u, mag, fused);
        // every u of a level must give the level's own magnitude
        if (F16::store(mag) != F16::store(mx_level_value<M>((int)lv))) atomicMax(&g_mx_bad[slot], 4);
        reinterpret_cast<uint8_t*>(tab)[i] = (uint8_t)lv;
    }
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

typedef _Float16 mx_h2_t __attribute__((ext_vector_type(2)));

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

// block max of the 16-bit patterns over the L lanes of a block (L = 2 or 4, aligned)
template <int L>
__device__ __forceinline__ uint32_t lanes_max(uint32_t v) {
    uint32_t o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xf, 0xf, true);   // quad_perm [1,0,3,2]
    v = v > o ? v : o;
    if constexpr (L == 4) {
        o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xf, 0xf, true);        // quad_perm [2,3,0,1]
        v = v > o ? v : o;
    }
    return v;
}

// float through a DPP move (quad_perm patterns below)
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}

// Persistent 512-thread workgroups; each wave takes 1024-element tiles (the lane
// mapping above).  BLK: block size 16 or 32.  n_elems is a multiple of BLK.
template <int M, int BLK>
__global__ __launch_bounds__(kMxThreads) void mx_fast_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
                                                             uint16_t* __restrict__ scales,
                                                             uint8_t* __restrict__ codes, int64_t n_elems, int slot,
                                                             int n, uint32_t lo_m1, MxParams p) {
    constexpr int LPB = BLK / 8;   // lanes of a block within a half
    typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
    typedef uint16_t u16x2_t __attribute__((ext_vector_type(2)));
    extern __shared__ __attribute__((aligned(16))) uint32_t tab[];
    const int lane = (int)(threadIdx.x & 63);
    const int wave = (int)(threadIdx.x >> 6);
    const int q = lane & 3;   // lane within its quad
    const bool lead = (lane & (LPB - 1)) == 0;
    const int64_t ntiles = (n_elems + 1023) / 1024;
    const int64_t stride = (int64_t)gridDim.x * (kMxThreads / 64);

    uint32_t w[2][4];
    auto load = [&](int64_t tile) __attribute__((always_inline)) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int64_t off = tile * 1024 + 512 * h + 8 * lane;
            if (tile < ntiles && off < n_elems) {   // whole 8-element chunks: n_elems % 16 == 0
                const u32x4_t a = *reinterpret_cast<const u32x4_t*>(x + off);
                w[h][0] = a.x; w[h][1] = a.y; w[h][2] = a.z; w[h][3] = a.w;
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) w[h][i] = 0u;
            }
        }
    };
    // the first tile's loads go out before the table copy, so their latency overlaps it
    int64_t tile = (int64_t)blockIdx.x * (kMxThreads / 64) + wave;
    load(tile);
    {   // copy the table in 16-byte pieces (the slot arrays are 16-byte aligned rows)
        const uint4* src = reinterpret_cast<const uint4*>(g_mx_tab[slot]);
        uint4* dst = reinterpret_cast<uint4*>(tab);
        for (int i = threadIdx.x; i < (n + 2 + 15) / 16; i += kMxThreads) dst[i] = src[i];
    }
    // the fp16 log2 thresholds of the shared scale, after the table
    float* l2t = reinterpret_cast<float*>(tab + (n + 2 + 15) / 16 * 4);
    for (int i = threadIdx.x; i < 80; i += kMxThreads) l2t[i] = i < 40 ? kLog2FloorF16[i] : kLog2RoundF16[i - 40];
    __syncthreads();
    const LdsLog2 lt{l2t, l2t + 40};

    for (; tile < ntiles; tile += stride) {
        int64_t off[2];
        bool valid[2];
        uint32_t m2[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            off[h] = tile * 1024 + 512 * h + 8 * lane;
            valid[h] = off[h] < n_elems;
            // block max of |x| over the 16-bit patterns (NaN patterns sort above inf)
            u16x2_t mp = __builtin_bit_cast(u16x2_t, w[h][0] & 0x7fff7fffu);
#pragma unroll
            for (int i = 1; i < 4; ++i)
                mp = __builtin_elementwise_max(mp, __builtin_bit_cast(u16x2_t, w[h][i] & 0x7fff7fffu));
            m2[h] = lanes_max<LPB>(mp.x > mp.y ? (uint32_t)mp.x : (uint32_t)mp.y);
        }
        // one shared-scale evaluation per lane: a quad holds 4 blocks (block 16: 2 per
        // half) or 2 (block 32: 1 per half); lane q scales block (half q >> 1, pair q & 1),
        // then every lane takes the scales of its two blocks from the lanes that made them
        float sm;
        if constexpr (BLK == 16) {
            const float a = dpp_f<0x88>(__builtin_bit_cast(float, m2[0]));   // quad_perm [0,2,0,2]
            const float b = dpp_f<0x88>(__builtin_bit_cast(float, m2[1]));
            sm = (q >> 1) ? b : a;
        } else {
            sm = (q >> 1) ? __builtin_bit_cast(float, m2[1]) : __builtin_bit_cast(float, m2[0]);
        }
        const float s_own = mx_shared_scale<F16>(F16::load((uint16_t)__builtin_bit_cast(uint32_t, sm)), p, lt);
        const float rs_own = 1.0f / s_own;
        float s[2], rs[2];
        if constexpr (BLK == 16) {
            s[0] = dpp_f<0x50>(s_own);   // quad_perm [0,0,1,1]
            s[1] = dpp_f<0xFA>(s_own);   // quad_perm [2,2,3,3]
            rs[0] = dpp_f<0x50>(rs_own);
            rs[1] = dpp_f<0xFA>(rs_own);
        } else {
            s[0] = dpp_f<0x00>(s_own);   // quad_perm [0,0,0,0]
            s[1] = dpp_f<0xAA>(s_own);   // quad_perm [2,2,2,2]
            rs[0] = dpp_f<0x00>(rs_own);
            rs[1] = dpp_f<0xAA>(rs_own);
        }
        const bool special = (m2[0] > 0x7c00u) | (m2[1] > 0x7c00u) | !(s_own > 0.f && s_own < __builtin_inff());

        uint32_t y2[2][4];
        uint32_t cout[2][8];
        const mx_h2_t s2h[2] = {(mx_h2_t){(_Float16)s[0], (_Float16)s[0]}, (mx_h2_t){(_Float16)s[1], (_Float16)s[1]}};
        if (__builtin_expect(__builtin_amdgcn_ballot_w64(special) != 0, 0)) {
            // a NaN in the wave's tile, or a scale that rounds to 0 or inf in fp16 (an
            // 8-bit scale exponent): the generic element path
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float o[2];
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const float v = F16::load((uint16_t)(e ? w[h][i] >> 16 : w[h][i] & 0xffffu));
                        const float yv = p.pot ? F16::round(v * rs[h]) : div_T<F16>(v, s[h], rs[h]);
                        o[e] = F16::round(elem_quant<F16, M>(yv, cout[h][2 * i + e], p.fused) * s[h]);
                    }
                    y2[h][i] = (uint32_t)F16::store(o[0]) | ((uint32_t)F16::store(o[1]) << 16);
                }
        } else {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                // u = R16(|x| / s) of each element, packed in pairs like x: for a power-of-two
                // scale the product is exact; for an FP scale R16(|x| * R32(1/s)) (one
                // rounding) equals R16(|x| / s) unless the quotient is below 2^-14
                uint32_t u2[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    u2[i] = mix_lo(w[h][i], rs[h]);
                    mix_hi(u2[i], w[h][i], rs[h]);
                }
                if (!p.pot) {
                    u16x2_t mn = __builtin_bit_cast(u16x2_t, u2[0]);
#pragma unroll
                    for (int i = 1; i < 4; ++i) mn = __builtin_elementwise_min(mn, __builtin_bit_cast(u16x2_t, u2[i]));
                    if ((mn.x <= 0x0400u) | (mn.y <= 0x0400u)) {   // near or in the subnormal range: divide
#pragma unroll
                        for (int i = 0; i < 8; ++i) {
                            const uint32_t key = i & 1 ? u2[i / 2] >> 16 : u2[i / 2] & 0xffffu;
                            if (key <= 0x0400u) {
                                const float a =
                                    fabsf(F16::load((uint16_t)(i & 1 ? w[h][i / 2] >> 16 : w[h][i / 2] & 0xffffu)));
                                const uint32_t k2 = F16::store(a / s[h]);
                                u2[i / 2] = i & 1 ? (u2[i / 2] & 0xffffu) | (k2 << 16) : (u2[i / 2] & 0xffff0000u) | k2;
                            }
                        }
                    }
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    uint32_t e2[2];
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const int key = (int)(e ? u2[i] >> 16 : u2[i] & 0xffffu);
                        int k;   // byte index k + 1 clamped to [0, n + 1] in one v_med3_i32
                        asm("v_med3_i32 %0, %1, 0, %2" : "=v"(k) : "v"(key - (int)lo_m1), "s"(n + 1));
                        e2[e] = reinterpret_cast<const uint8_t*>(tab)[k];
                    }
                    // the level values from the level codes lv = e << M | m, both halves at once:
                    // F = fp16 bits (lv << (10 - M)) + (14 << 10) is (1 + m / 2^M) * 2^(e - 1), the
                    // value for e >= 1; for e = 0 it is 1/2 + m / 2^(M + 1) and the value m / 2^M
                    // is 2F - 1 (exact).  2F - 1 < F exactly when F < 1, i.e. e = 0, so the value
                    // is min(F, 2F - 1) in both cases.
                    const uint32_t l2v = e2[0] | (e2[1] << 16);
                    const mx_h2_t F = __builtin_bit_cast(mx_h2_t, (l2v << (10 - M)) + 0x38003800u);
                    const mx_h2_t two = {(_Float16)2.0f, (_Float16)2.0f}, mone = {(_Float16)-1.0f, (_Float16)-1.0f};
                    const uint32_t q2 = __builtin_bit_cast(uint32_t, __builtin_elementwise_min(F, __builtin_elementwise_fma(F, two, mone)));
                    // R16(q * s) of both: s is an fp16 value here, so v_pk_mul_f16 rounds the
                    // exact products once
                    const uint32_t o2 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(mx_h2_t, q2) * s2h[h]);
                    // the sign of x unless u is +-0 (the reference's u == 0 gives +0 and code 0):
                    // bit 15 of each half of u2 + 0x7fff7fff is set iff that half is nonzero
                    // (u <= 0x7c00, so no carry crosses the halves)
                    const uint32_t sg = w[h][i] & (u2[i] + 0x7fff7fffu) & 0x80008000u;
                    y2[h][i] = o2 | sg;
                    cout[h][2 * i] = (e2[0] & 0xffu) | (((sg >> 15) & 1u) << (M + 2));
                    cout[h][2 * i + 1] = (e2[1] & 0xffu) | ((sg >> 31) << (M + 2));
                }
            }
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            if (!valid[h]) continue;
            *reinterpret_cast<u32x4_t*>(y + off[h]) = (u32x4_t){y2[h][0], y2[h][1], y2[h][2], y2[h][3]};
            if (codes) {
                if constexpr (M == 1) {
                    uint32_t c = 0;
#pragma unroll
                    for (int i = 0; i < 8; ++i) c |= (cout[h][i] & 0xfu) << (4 * i);
                    *reinterpret_cast<uint32_t*>(codes + off[h] / 2) = c;
                } else {
                    uint32_t c0 = 0, c1 = 0;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        c0 |= (cout[h][i] & 0xffu) << (8 * i);
                        c1 |= (cout[h][4 + i] & 0xffu) << (8 * i);
                    }
                    *reinterpret_cast<uint2*>(codes + off[h]) = make_uint2(c0, c1);
                }
            }
            if (scales != nullptr && lead) scales[off[h] / BLK] = F16::store(s[h]);
        }
        load(tile + stride);
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

template <int M, int BLK>
int launch_mx_fast(const void* x, void* y, void* scales, void* codes, int64_t n_elems, int slot, int n,
                   uint32_t lo_bits, const MxParams& p, int dev, hipStream_t st) {
    const size_t lds = (size_t)((n + 2 + 15) / 16) * 16 + 80 * sizeof(float);
    auto kern = mx_fast_kernel<M, BLK>;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kMxThreads, lds) != hipSuccess || per_cu <= 0)
        return 0;
    const int64_t ntiles = (n_elems + 1023) / 1024;
    const int64_t waves_needed = ntiles;
    // twice the waves that fit at once: the workgroups beyond them start as the first ones
    // finish, which staggers the waves' load / compute phases (configs[1]: 2 tiles a wave
    // instead of 3; MXFP4 17.7 -> 16.9 us, NVFP4 18.6 -> 17.4 us, MXFP8 within 1%)
    const int64_t resident = 2 * (int64_t)g_mx_cus[dev] * per_cu * (kMxThreads / 64);
    // as many rounds as those waves need, with the tiles spread evenly over them
    const int64_t rounds = (waves_needed + resident - 1) / resident;
    const int64_t waves = (waves_needed + rounds - 1) / rounds;
    const int64_t grid = (waves + kMxThreads / 64 - 1) / (kMxThreads / 64);
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(kMxThreads), lds, st, (const uint16_t*)x, (uint16_t*)y,
                       (uint16_t*)scales, (uint8_t*)codes, n_elems, slot, n, lo_bits - 1u, p);
    return 1;
}

template <int M>
int mx_fast_block(int block, const void* x, void* y, void* scales, void* codes, int64_t n_elems, int slot, int n,
                  uint32_t lo_bits, const MxParams& p, int dev, hipStream_t st) {
    if (block == 16) return launch_mx_fast<M, 16>(x, y, scales, codes, n_elems, slot, n, lo_bits, p, dev, st);
    return launch_mx_fast<M, 32>(x, y, scales, codes, n_elems, slot, n, lo_bits, p, dev, st);
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
    const int64_t n_elems = rows * cols;
    if (n_elems == 0) return 1;
    switch (mbit) {
        case 1: return mx_fast_block<1>(block, x, y, scales, codes, n_elems, slot, n, lo_bits, p, dev, st);
        case 2: return mx_fast_block<2>(block, x, y, scales, codes, n_elems, slot, n, lo_bits, p, dev, st);
        case 3: return mx_fast_block<3>(block, x, y, scales, codes, n_elems, slot, n, lo_bits, p, dev, st);
        default: return mx_fast_block<5>(block, x, y, scales, codes, n_elems, slot, n, lo_bits, p, dev, st);
    }
}
