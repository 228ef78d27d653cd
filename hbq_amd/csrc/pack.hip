// Packed HBQ tensors: the bit-level wire format of the HBQ quantizer's outputs
// and its exact decoder.
//
// For x [rows, cols] quantized with block B, l2 block b, element format E2Mm and
// L2 index width w, a row packs into four byte strings:
//   codes:  cols fields of m + 3 bits (sign | 2-bit exponent | m mantissa bits),
//           element i at bits [(m+3) i, (m+3)(i+1)) of the little-endian bit string
//           (the element order of LP_DATA in hardware/HBQ_accelerator/
//           hbq_e_quantizer/top.sv:40-45 and of the MAC vectors, tb_WXAY.sv:174-180)
//   l1:     one E5M3 byte per block: exponent field (bias 15) << 3 | mantissa
//           (SCALE_EXP_BIAS 15 / SCALE_MANT 3 of top.sv:23-26): bits [14:7] of the
//           scale as fp16; 0xFF marks a scale that is not a finite E5M3 number
//   l2:     w bits per sub-block, LSB first (L2_SCALE bit i = micro-block i, top.sv:44)
//   scheme: one bit per block, LSB first (Mix only)
// Decoding computes the reference's dequantization d = R(R(q l2[j][s]) l1)
// (src/quantizer.py:790-796) from the level q of each code, so unpack(pack(...))
// reproduces the quantizer's output bit for bit.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <type_traits>

#include "hbq_capi_internal.h"
#include "quant_common.h"

namespace hbq {
namespace {

// R_T(level value * l2[j][s]) for every scheme s, candidate j and level (block
// independent), rounded on the host; indexed [(s * 8 + j) * 32 + level]
struct UnpackParams {
    float qs[2 * kMaxJ * 32];
};

// E5M3 byte of a scale held in T (0xFF if it is not a finite E5M3 value)
template <class T>
__device__ __forceinline__ uint32_t e5m3_byte(typename T::storage s) {
    const float v = T::load(s);
    const uint32_t b = f2bits(v);
    if (b == 0) return 0;                                            // +0: mantissa 0 of the subnormal range
    if (!(v > 0.f) || v > 61440.f) return 0xffu;                   // NaN, inf, < 0, out of range
    if (v < 0x1p-14f) {                                              // E5M3 subnormal m / 8 * 2^-14
        const float m = v * 0x1p17f;
        return (m == (float)(int)m && m < 8.f) ? (uint32_t)m : 0xffu;
    }
    if (b & 0xfffffu) return 0xffu;                                  // more than 3 mantissa bits
    return ((((b >> 23) & 0xffu) - 127u + 15u) << 3) | ((b >> 20) & 7u);
}

__device__ __forceinline__ float e5m3_value(uint32_t byte) {
    const uint32_t e = byte >> 3, m = byte & 7u;
    if (e == 31) return __builtin_nanf("");
    if (e == 0) return (float)m * 0x1p-17f;
    return bits2f(((e - 15u + 127u) << 23) | (m << 20));
}

// thread = (row, 8 elements): quantizer codes -> (M+3)-bit fields
template <int M>
__global__ __launch_bounds__(kThreads) void pack_codes_kernel(const uint8_t* __restrict__ in, uint8_t* __restrict__ out,
                                                              int64_t rows, int64_t cols) {
    constexpr int W = M + 3;
    const int64_t groups = cols / 8;
    const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (t >= rows * groups) return;
    const int64_t r = t / groups, g = t - r * groups;
    uint64_t acc = 0;
    if constexpr (M == 1) {
        acc = *reinterpret_cast<const uint32_t*>(in + r * (cols / 2) + g * 4);   // already two per byte
    } else {
        const u32x2 v = *reinterpret_cast<const u32x2*>(in + r * cols + g * 8);
        const uint64_t w = (uint64_t)v.x | ((uint64_t)v.y << 32);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc |= ((w >> (8 * i)) & ((1u << W) - 1u)) << (W * i);
    }
    uint8_t* o = out + r * (cols * W / 8) + g * W;
    if constexpr (M == 1) {
        *reinterpret_cast<uint32_t*>(o) = (uint32_t)acc;
    } else {
#pragma unroll
        for (int i = 0; i < W; ++i) o[i] = (uint8_t)(acc >> (8 * i));
    }
}

// fields of `w` bits (one per input byte, n per row) -> LSB-first bit strings of
// `ob` bytes per row; thread = output byte
__global__ __launch_bounds__(kThreads) void pack_bits_kernel(const uint8_t* __restrict__ in, uint8_t* __restrict__ out,
                                                             int64_t rows, int64_t n, int w, int64_t ob) {
    const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (t >= rows * ob) return;
    const int64_t r = t / ob, j = t - r * ob;
    uint32_t byte = 0;
    for (int b = 0; b < 8; ++b) {
        const int64_t p = j * 8 + b, f = p / w;
        if (f >= n) break;
        byte |= ((uint32_t)(in[r * n + f] >> (p - f * w)) & 1u) << b;
    }
    out[t] = (uint8_t)byte;
}

template <class T>
__global__ __launch_bounds__(kThreads) void pack_l1_kernel(const typename T::storage* __restrict__ l1,
                                                           uint8_t* __restrict__ out, int64_t n) {
    const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (t < n) out[t] = (uint8_t)e5m3_byte<T>(l1[t]);
}

// bits [pos, pos + w) of a row's LSB-first bit string (w <= 3, so at most two bytes)
__device__ __forceinline__ uint32_t get_bits(const uint8_t* __restrict__ row, int64_t pos, int w, int64_t row_bytes) {
    const int64_t byte = pos >> 3;
    uint32_t v = row[byte];
    if (byte + 1 < row_bytes) v |= (uint32_t)row[byte + 1] << 8;
    return (v >> (pos & 7)) & ((1u << w) - 1u);
}

// Decode: a workgroup copies the block-independent magnitudes R(level * l2[j][s])
// to LDS; a thread decodes 8 consecutive elements of one row (one block, at most
// two sub-blocks): per element one LDS read, then d = R(m * l1) and the code's sign.
// fp16 multiplies pairs with v_pk_mul_f16 (one rounding of the exact product of
// two fp16 values, as R16(m * l1) needs); bf16 multiplies in fp32 and rounds a
// pair with one v_cvt_pk_bf16_f32.
template <class T, int M>
__global__ __launch_bounds__(kThreads) void unpack_kernel(const uint8_t* __restrict__ pc, const uint8_t* __restrict__ pl1,
                                                          const uint8_t* __restrict__ pl2, const uint8_t* __restrict__ ps,
                                                          typename T::storage* __restrict__ y, int64_t rows, int64_t cols,
                                                          int block, int l2b, int l2bits, int S, UnpackParams p) {
    constexpr int W = M + 3;
    constexpr int L = 1 << (M + 2);
    constexpr bool H = sizeof(typename T::storage) == 2 && T::dt == kF16;
    using E = typename std::conditional<H, _Float16, float>::type;
    __shared__ E tab[2 * kMaxJ * L];
    for (int i = threadIdx.x; i < 2 * kMaxJ * L; i += kThreads) tab[i] = (E)p.qs[(i / L) * 32 + (i % L)];
    __syncthreads();

    const int64_t groups = cols / 8;
    const int64_t g = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (g >= groups) return;
    const int64_t nblk = cols / block;
    const int64_t l2_row = (cols / l2b * l2bits + 7) / 8;
    const int64_t c0 = g * 8, blk = c0 / block;
#pragma unroll 2
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
        const float l1 = e5m3_value(pl1[r * nblk + blk]);
        const int s = S == 2 ? (ps[r * ((nblk + 7) / 8) + (blk >> 3)] >> (blk & 7)) & 1 : 0;
        // candidates of the (one or two) sub-blocks of these 8 elements
        int j0 = 0, j1 = 0;
        if (l2bits) {
            const uint8_t* l2r = pl2 + r * l2_row;
            j0 = (int)get_bits(l2r, c0 / l2b * l2bits, l2bits, l2_row);
            j1 = l2b >= 8 ? j0 : (int)get_bits(l2r, (c0 + 4) / l2b * l2bits, l2bits, l2_row);
        }
        const E* t0 = tab + (s * kMaxJ + j0) * L;
        const E* t1 = tab + (s * kMaxJ + j1) * L;

        uint64_t acc = 0;
        const uint8_t* src = pc + r * (cols * W / 8) + g * W;
        if constexpr (M == 1) {
            acc = *reinterpret_cast<const uint32_t*>(src);
        } else {
#pragma unroll
            for (int i = 0; i < W; ++i) acc |= (uint64_t)src[i] << (8 * i);
        }
        uint32_t w[4];
        if constexpr (H) {
            typedef _Float16 h2 __attribute__((ext_vector_type(2)));
            const _Float16 l1h = (_Float16)l1;   // an E5M3 value: exact in fp16
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t ca = (uint32_t)(acc >> (W * 2 * k)) & ((1u << W) - 1u);
                const uint32_t cb = (uint32_t)(acc >> (W * (2 * k + 1))) & ((1u << W) - 1u);
                const E* tk = k < 2 ? t0 : t1;
                const h2 m = {tk[ca & (L - 1)], tk[cb & (L - 1)]};
                const h2 d = m * (h2){l1h, l1h};
                asm volatile("" : : "v"(d));
                w[k] = __builtin_bit_cast(uint32_t, d) | ((ca >> (M + 2)) << 15) | ((cb >> (M + 2)) << 31);
            }
        } else if constexpr (sizeof(typename T::storage) == 2) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t ca = (uint32_t)(acc >> (W * 2 * k)) & ((1u << W) - 1u);
                const uint32_t cb = (uint32_t)(acc >> (W * (2 * k + 1))) & ((1u << W) - 1u);
                const E* tk = k < 2 ? t0 : t1;
                const bf16x2_t d = __builtin_convertvector((f32x2_t){tk[ca & (L - 1)] * l1, tk[cb & (L - 1)] * l1},
                                                           bf16x2_t);
                w[k] = __builtin_bit_cast(uint32_t, d) | ((ca >> (M + 2)) << 15) | ((cb >> (M + 2)) << 31);
            }
        }
        typename T::storage* dst = y + r * cols + c0;
        if constexpr (sizeof(typename T::storage) == 2) {
            *reinterpret_cast<u32x4*>(dst) = (u32x4){w[0], w[1], w[2], w[3]};
        } else {
            float out[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t c = (uint32_t)(acc >> (W * i)) & ((1u << W) - 1u);
                const float d = (i < 4 ? t0 : t1)[c & (L - 1)] * l1;
                out[i] = bits2f(f2bits(d) | ((c >> (M + 2)) << 31));
            }
            *reinterpret_cast<f32x4*>(dst) = (f32x4){out[0], out[1], out[2], out[3]};
            *reinterpret_cast<f32x4*>(dst + 4) = (f32x4){out[4], out[5], out[6], out[7]};
        }
    }
}

unsigned grid_for(int64_t n) { return (unsigned)((n + kThreads - 1) / kThreads); }

// round an exactly representable-in-double value to the dtype (RNE), on the host
float round_to(double v, int dt) {
    float f = (float)v;   // exact: a level times an L2 factor has few significant bits
    if (dt == kF16) return (float)(_Float16)f;
    if (dt == kBF16) {
        uint32_t x;
        memcpy(&x, &f, 4);
        x += 0x7fffu + ((x >> 16) & 1u);
        x &= 0xffff0000u;
        memcpy(&f, &x, 4);
    }
    return f;
}

// shared argument checks; fills the row strides
int check_geometry(int64_t rows, int64_t cols, int dtype, int block, int mbit, int l2b, int l2_sc_bit, int l2_scheme,
                   int64_t strides[4]) {
    if (dtype != kF16 && dtype != kBF16 && dtype != kF32) return hbq_fail(HBQ_ERR_INVALID, "bad dtype code %d", dtype);
    if (rows < 0 || cols < 0) return hbq_fail(HBQ_ERR_INVALID, "negative size");
    if (mbit < 1 || mbit > 3) return hbq_fail(HBQ_ERR_UNSUPPORTED, "packed codes need mbit 1..3, got %d", mbit);
    if (block < 8 || block % 8) return hbq_fail(HBQ_ERR_UNSUPPORTED, "packed blocks need block_size % 8 == 0");
    if (l2b <= 0 || block % l2b) return hbq_fail(HBQ_ERR_INVALID, "block_size must be divisible by l2_block_size");
    if (cols % block) return hbq_fail(HBQ_ERR_UNSUPPORTED, "packed rows need cols %% block_size == 0");
    if (l2_sc_bit < 0 || l2_sc_bit > 3) return hbq_fail(HBQ_ERR_UNSUPPORTED, "l2_sc_bit %d not in 0..3", l2_sc_bit);
    if (l2_scheme < 0 || l2_scheme > 7) return hbq_fail(HBQ_ERR_INVALID, "Invalid L2 scheme code %d", l2_scheme);
    const int64_t nblk = cols / block;
    strides[0] = cols * (mbit + 3) / 8;
    strides[1] = nblk;
    strides[2] = (cols / l2b * l2_sc_bit + 7) / 8;
    strides[3] = l2_scheme == 7 ? (nblk + 7) / 8 : 0;
    return 0;
}

}  // namespace
}  // namespace hbq

using namespace hbq;

extern "C" {

int hbq_hbq_packed_strides(int64_t cols, int block_size, int mbit, int l2_block_size, int l2_sc_bit, int l2_scheme,
                           int64_t* strides) {
    hbq_clear_error();
    if (strides == nullptr) return hbq_fail(HBQ_ERR_INVALID, "null strides");
    return check_geometry(0, cols, kF16, block_size, mbit, l2_block_size, l2_sc_bit, l2_scheme, strides);
}

int hbq_hbq_pack(const void* codes, const void* l1_scale, const void* l2_index, const void* scheme, void* pcodes,
                 void* pl1, void* pl2, void* pscheme, int64_t rows, int64_t cols, int dtype, int block_size, int mbit,
                 int l2_block_size, int l2_sc_bit, int l2_scheme, void* stream) {
    hbq_clear_error();
    int64_t st4[4];
    if (int rc = check_geometry(rows, cols, dtype, block_size, mbit, l2_block_size, l2_sc_bit, l2_scheme, st4))
        return rc;
    if (rows == 0 || cols == 0) return 0;
    if (!codes || !l1_scale || !pcodes || !pl1) return hbq_fail(HBQ_ERR_INVALID, "null codes or scale pointer");
    if (l2_sc_bit > 0 && (!l2_index || !pl2)) return hbq_fail(HBQ_ERR_INVALID, "null L2 index pointer");
    if (l2_scheme == 7 && (!scheme || !pscheme)) return hbq_fail(HBQ_ERR_INVALID, "null scheme pointer");
    if (((uintptr_t)codes | (uintptr_t)pcodes) % 8) return hbq_fail(HBQ_ERR_INVALID, "code buffers must be 8-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    const int64_t groups = rows * (cols / 8);
    if (mbit == 1)
        hipLaunchKernelGGL(pack_codes_kernel<1>, dim3(grid_for(groups)), dim3(kThreads), 0, st, (const uint8_t*)codes,
                           (uint8_t*)pcodes, rows, cols);
    else if (mbit == 2)
        hipLaunchKernelGGL(pack_codes_kernel<2>, dim3(grid_for(groups)), dim3(kThreads), 0, st, (const uint8_t*)codes,
                           (uint8_t*)pcodes, rows, cols);
    else
        hipLaunchKernelGGL(pack_codes_kernel<3>, dim3(grid_for(groups)), dim3(kThreads), 0, st, (const uint8_t*)codes,
                           (uint8_t*)pcodes, rows, cols);
    const int64_t nb = rows * st4[1];
    if (dtype == kF16)
        hipLaunchKernelGGL(pack_l1_kernel<F16>, dim3(grid_for(nb)), dim3(kThreads), 0, st, (const uint16_t*)l1_scale,
                           (uint8_t*)pl1, nb);
    else if (dtype == kBF16)
        hipLaunchKernelGGL(pack_l1_kernel<BF16>, dim3(grid_for(nb)), dim3(kThreads), 0, st, (const uint16_t*)l1_scale,
                           (uint8_t*)pl1, nb);
    else
        hipLaunchKernelGGL(pack_l1_kernel<F32>, dim3(grid_for(nb)), dim3(kThreads), 0, st, (const float*)l1_scale,
                           (uint8_t*)pl1, nb);
    if (l2_sc_bit > 0)
        hipLaunchKernelGGL(pack_bits_kernel, dim3(grid_for(rows * st4[2])), dim3(kThreads), 0, st,
                           (const uint8_t*)l2_index, (uint8_t*)pl2, rows, cols / l2_block_size, l2_sc_bit, st4[2]);
    if (l2_scheme == 7)
        hipLaunchKernelGGL(pack_bits_kernel, dim3(grid_for(rows * st4[3])), dim3(kThreads), 0, st,
                           (const uint8_t*)scheme, (uint8_t*)pscheme, rows, st4[1], 1, st4[3]);
    return hbq_check_launch("hbq_hbq_pack");
}

int hbq_hbq_unpack(const void* pcodes, const void* pl1, const void* pl2, const void* pscheme, void* y, int64_t rows,
                   int64_t cols, int dtype, int block_size, int mbit, int l2_block_size, int l2_sc_bit, int l2_scheme,
                   void* stream) {
    hbq_clear_error();
    int64_t st4[4];
    if (int rc = check_geometry(rows, cols, dtype, block_size, mbit, l2_block_size, l2_sc_bit, l2_scheme, st4))
        return rc;
    if (rows == 0 || cols == 0) return 0;
    if (!pcodes || !pl1 || !y) return hbq_fail(HBQ_ERR_INVALID, "null codes, scale or output pointer");
    if (l2_sc_bit > 0 && !pl2) return hbq_fail(HBQ_ERR_INVALID, "null L2 index pointer");
    if (l2_scheme == 7 && !pscheme) return hbq_fail(HBQ_ERR_INVALID, "null scheme pointer");
    if ((uintptr_t)pcodes % 8 || (uintptr_t)y % 16) return hbq_fail(HBQ_ERR_INVALID, "misaligned codes or output");
    HbqParams hp{};
    int S = 1;
    if (int rc = hbq_l2_table(hp, S, l2_sc_bit, l2_scheme, dtype)) return rc;
    UnpackParams p{};
    for (int s = 0; s < 2; ++s)
        for (int j = 0; j < kMaxJ; ++j)
            for (int lev = 0; lev < 32; ++lev) {
                const int e = lev >> mbit, m = lev & ((1 << mbit) - 1);
                const double lv = e == 0 ? ldexp((double)m, -mbit) : ldexp(1.0 + ldexp((double)m, -mbit), e - 1);
                const double l2 = j < hp.J ? hp.l2[j][s] : 1.0;
                p.qs[(s * kMaxJ + j) * 32 + lev] = lev < (4 << mbit) ? round_to(lv * l2, dtype) : 0.f;
            }
    hipStream_t st = (hipStream_t)stream;
    const int64_t groups = cols / 8;
    if (groups > 0x7fffffffll * kThreads) return hbq_fail(HBQ_ERR_INVALID, "rows too long");
    // about 2048 workgroups (8 per CU), each walking rows: the LDS table is built once per workgroup
    const int64_t gx = grid_for(groups);
    int64_t gy = 2048 / gx;
    gy = gy < 1 ? 1 : (gy > rows ? rows : (gy > 65535 ? 65535 : gy));
    const dim3 grid((unsigned)gx, (unsigned)gy);
#define UNPACK(TT, MM)                                                                                             \
    hipLaunchKernelGGL((unpack_kernel<TT, MM>), grid, dim3(kThreads), 0, st, (const uint8_t*)pcodes,              \
                       (const uint8_t*)pl1, (const uint8_t*)pl2, (const uint8_t*)pscheme, (TT::storage*)y, rows, cols, \
                       block_size, l2_block_size, l2_sc_bit, S, p)
#define UNPACK_M(TT) \
    if (mbit == 1) UNPACK(TT, 1); else if (mbit == 2) UNPACK(TT, 2); else UNPACK(TT, 3)
    if (dtype == kF16) { UNPACK_M(F16); }
    else if (dtype == kBF16) { UNPACK_M(BF16); }
    else { UNPACK_M(F32); }
#undef UNPACK_M
#undef UNPACK
    return hbq_check_launch("hbq_hbq_unpack");
}

}  // extern "C"
