// Device helpers shared by the quantizer kernels (quant.hip, hbq_fast.hip):
// 16-element lane loads/stores, code packing, block reductions and the
// reference's fp32 summation order for the HBQ scheme error.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hbq_numeric.h"

namespace hbq {

constexpr int kV = 16;          // elements per lane
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;   // 4 wavefronts per workgroup

template <class T>
__device__ __forceinline__ void load16(const typename T::storage* __restrict__ p, float* v) {
    if constexpr (sizeof(typename T::storage) == 2) {
        const u32x4* q = reinterpret_cast<const u32x4*>(p);
        u32x4 a = __builtin_nontemporal_load(q);
        u32x4 b = __builtin_nontemporal_load(q + 1);
        uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v[2 * i] = T::load((uint16_t)(w[i] & 0xffffu));
            v[2 * i + 1] = T::load((uint16_t)(w[i] >> 16));
        }
    } else {
        const f32x4* q = reinterpret_cast<const f32x4*>(p);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f32x4 a = __builtin_nontemporal_load(q + i);
            v[4 * i] = a.x; v[4 * i + 1] = a.y; v[4 * i + 2] = a.z; v[4 * i + 3] = a.w;
        }
    }
}

template <class T>
__device__ __forceinline__ void store16(typename T::storage* __restrict__ p, const float* v) {
    if constexpr (sizeof(typename T::storage) == 2) {
        uint32_t w[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if constexpr (T::dt == kBF16) {   // one v_cvt_pk_bf16_f32 per pair
                w[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){v[2 * i], v[2 * i + 1]}, bf16x2_t));
            } else {
                w[i] = (uint32_t)T::store(v[2 * i]) | ((uint32_t)T::store(v[2 * i + 1]) << 16);
            }
        }
        u32x4* q = reinterpret_cast<u32x4*>(p);
        __builtin_nontemporal_store((u32x4){w[0], w[1], w[2], w[3]}, q);
        __builtin_nontemporal_store((u32x4){w[4], w[5], w[6], w[7]}, q + 1);
    } else {
        f32x4* q = reinterpret_cast<f32x4*>(p);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_nontemporal_store((f32x4){v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]}, q + i);
    }
}

// Codes of 16 consecutive elements starting at column c0 (a multiple of 16).
// 4-bit formats pack two codes per byte (even column in the low nibble) with a
// row stride of ceil(cols/2) bytes; wider formats use one byte per element.
template <int M>
__device__ __forceinline__ void store_codes(uint8_t* __restrict__ codes, int64_t row, int64_t cols, int64_t c0,
                                            const uint32_t* c, bool RAGGED) {
    if (codes == nullptr) return;
    if constexpr (M == 1) {
        const int64_t stride = (cols + 1) / 2;
        uint8_t* p = codes + row * stride + c0 / 2;
        if (!RAGGED) {
            uint32_t w0 = 0, w1 = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                w0 |= (c[i] & 0xfu) << (4 * i);
                w1 |= (c[8 + i] & 0xfu) << (4 * i);
            }
            *reinterpret_cast<uint2*>(p) = make_uint2(w0, w1);
        } else {
#pragma unroll
            for (int i = 0; i < 16; i += 2) {
                if (c0 + i >= cols) break;
                uint32_t hi = (c0 + i + 1 < cols) ? (c[i + 1] & 0xfu) : 0u;
                p[i / 2] = (uint8_t)((c[i] & 0xfu) | (hi << 4));
            }
        }
    } else {
        uint8_t* p = codes + row * cols + c0;
        if (!RAGGED) {
            uint32_t w[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                w[i] = (c[4 * i] & 0xffu) | ((c[4 * i + 1] & 0xffu) << 8) | ((c[4 * i + 2] & 0xffu) << 16) |
                       ((c[4 * i + 3] & 0xffu) << 24);
            *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i)
                if (c0 + i < cols) p[i] = (uint8_t)c[i];
        }
    }
}

// max of |x| bit patterns over a group of `lpb` lanes (NaN patterns order above +inf)
__device__ __forceinline__ uint32_t group_max_bits(uint32_t v, int lpb) {
    for (int off = 1; off < lpb; off <<= 1) {
        uint32_t o = (uint32_t)__shfl_xor((int)v, off, 64);
        v = v > o ? v : o;
    }
    return v;
}

// max over the 8 lanes of a block with DPP: swap neighbours, swap pairs, mirror halves of 8
__device__ __forceinline__ uint32_t max8_dpp(uint32_t v) {
    uint32_t o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xf, 0xf, true);   // quad_perm [1,0,3,2]
    v = v > o ? v : o;
    o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xf, 0xf, true);            // quad_perm [2,3,0,1]
    v = v > o ? v : o;
    o = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xf, 0xf, true);           // row_half_mirror
    return v > o ? v : o;
}

struct Locate {
    int64_t gb;     // global block index
    int li;         // lane within the block
    bool valid;
    int64_t row, c0;
};

__device__ __forceinline__ Locate locate(int lpb_log2, int64_t nblk_row, int64_t nb, int block) {
    Locate L;
    int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    L.gb = t >> lpb_log2;
    L.li = (int)(threadIdx.x & ((1 << lpb_log2) - 1));
    L.valid = L.gb < nb;
    int64_t g = L.valid ? L.gb : 0;
    L.row = g / nblk_row;
    L.c0 = (g - L.row * nblk_row) * block + (int64_t)L.li * kV;
    return L;
}

template <class T>
__device__ __forceinline__ void load_lane(const typename T::storage* __restrict__ x, const Locate& L, int64_t cols,
                                          float* v, bool RAGGED) {
    if (!RAGGED) {
        if (L.valid) load16<T>(x + L.row * cols + L.c0, v);
        else {
#pragma unroll
            for (int i = 0; i < kV; ++i) v[i] = 0.f;
        }
    } else {
#pragma unroll
        for (int i = 0; i < kV; ++i) {
            int64_t c = L.c0 + i;
            v[i] = (L.valid && c < cols) ? T::load(x[L.row * cols + c]) : 0.f;
        }
    }
}

template <class T>
__device__ __forceinline__ void store_lane(typename T::storage* __restrict__ y, const Locate& L, int64_t cols,
                                           const float* v, bool RAGGED) {
    if (!L.valid) return;
    if (!RAGGED) {
        store16<T>(y + L.row * cols + L.c0, v);
    } else {
#pragma unroll
        for (int i = 0; i < kV; ++i) {
            int64_t c = L.c0 + i;
            if (c < cols) y[L.row * cols + c] = T::store(v[i]);
        }
    }
}

constexpr int kMaxJ = 8;

// MXFP / NVFP parameters (MXFPQuantizer, src/quantizer.py:430-511)
struct MxParams {
    int pot;              // 1: power-of-two scale (sc_mbit == 0), 0: FP scale
    int use_round;
    float ele_emax;       // 2^(ebit-1)
    float sc_emin, sc_emax;
    float min_normal;     // added to an all-zero block before log2
    float ele_maxnorm;    // element max normal (FP scale divisor)
    ScaleFmt sf;          // FP scale format
    int per_tensor;
    float tscale;         // per-tensor scale, already rounded to T
    int fused;            // element rounding of the compiled lpfp_quant (activate_dynamo=True)
};

template <class T, class Tab = ConstLog2>
__device__ __forceinline__ float mx_shared_scale(float amax, const MxParams& p, Tab tab = Tab()) {
    if (p.pot) {
        float v = T::round(amax + (amax == 0.f ? p.min_normal : 0.f));
        float se;
        if (v != v) se = v;
        else if (v == __builtin_inff()) se = __builtin_inff();
        else se = log2_exponent<T>(v, p.use_round, tab);
        se = T::round(se - p.ele_emax);
        se = se < p.sc_emin ? p.sc_emin : (se > p.sc_emax ? p.sc_emax : se);
        if (se != se) return se;
        return T::round(pow2f((int)se));
    }
    return scale_quant<T>(T::round(amax / p.ele_maxnorm), p.sf, tab);
}

struct HbqParams {
    int J;                       // number of L2 candidates (2^l2_sc_bit)
    float l2[kMaxJ][2];          // L2 factors per candidate and scheme, in T
    float rl2[kMaxJ][2];         // correctly rounded reciprocals
    float em[2];                 // R_T(ele_max * max_j l2[j, s])
    ScaleFmt sf;                 // E5M3 L1 scale format
    int fused;                   // element rounding of the compiled lpfp_quant (use_quant_kernel=True)
};

// Host: the L2 candidate factors of a scheme (HBQ_L2_* code) rounded to the
// dtype, and S (2 for Mix, else 1); 0 or an HBQ_ERR_* code.
int hbq_l2_table(HbqParams& p, int& S, int l2_sc_bit, int l2_scheme, int dtype);

// v replaces best (torch.argmin order: NaN is the smallest, the first minimum wins):
// v < best, or v NaN and best not.  !(v >= best) is v < best or either NaN.
__device__ __forceinline__ bool better(float v, float best) { return !(v >= best) & (best == best); }

// torch's fp32 order for the block error of one scheme (four interleaved
// cascades over the 128.. elements, combined left to right), computed by the
// lanes of one block.  sq holds this lane's 16 squared errors.
__device__ __forceinline__ float block_row_sum(const float* sq, int li, int lpb, int lane_base) {
    const int cl = lpb < 4 ? lpb : 4;                 // lanes per 16-term chunk
    float run[4] = {0.f, 0.f, 0.f, 0.f};
    for (int step = 0; step < cl; ++step) {
        float prev[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) prev[k] = __shfl_up(run[k], 1, 64);
        if ((li % cl) == step) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                float a = step == 0 ? 0.f : prev[k];
                a += sq[k];
                a += sq[k + 4];
                a += sq[k + 8];
                a += sq[k + 12];
                run[k] = a;
            }
        }
    }
    const int nchunks = lpb / cl;
    float P[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) P[k] = __shfl(run[k], lane_base + cl - 1, 64);
    for (int c = 1; c < nchunks; ++c) {
#pragma unroll
        for (int k = 0; k < 4; ++k) P[k] += __shfl(run[k], lane_base + c * cl + cl - 1, 64);
    }
    return ((P[0] + P[1]) + P[2]) + P[3];
}

// block_row_sum for blocks of 8 lanes (the table kernels' layout; blocks start at a
// multiple of 8 lanes): the same additions in the same order, with DPP moves in
// place of the lane shuffles
template <int CTRL>
__device__ __forceinline__ float dpp_movf(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}
__device__ __forceinline__ float block_row_sum8(const float* sq, int li) {
    float run[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int step = 0; step < 4; ++step) {
        float prev[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) prev[k] = dpp_movf<0x111>(run[k]);   // row_shr:1, lane - 1
        if ((li & 3) == step) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                float a = step == 0 ? 0.f : prev[k];
                a += sq[k];
                a += sq[k + 4];
                a += sq[k + 8];
                a += sq[k + 12];
                run[k] = a;
            }
        }
    }
    float P[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        // quad_perm [3,3,3,3]: lanes 0-3 of the block hold lane 3's cascade, 4-7 lane 7's;
        // row_half_mirror (lane i from lane 7 - i) brings the other one: the two-term sum
        // is the same in every lane since a + b == b + a
        const float q = dpp_movf<0xff>(run[k]);
        P[k] = q + dpp_movf<0x141>(q);
    }
    return ((P[0] + P[1]) + P[2]) + P[3];
}

}  // namespace hbq
