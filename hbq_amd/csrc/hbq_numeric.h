// Device-side numerics shared by the quantizer kernels.
//
// Every quantizer step of the reference is one PyTorch tensor op whose result
// is rounded to the tensor dtype T (fp16, bf16 or fp32).  The helpers here
// reproduce each step with one IEEE round-to-nearest-even to T.  This file is
// compiled with -ffp-contract=off: a fused multiply-add anywhere below would
// change results.
#pragma once
#include <type_traits>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "log2_tables.h"

namespace hbq {

enum DType : int { kF16 = 0, kBF16 = 1, kF32 = 2 };

__device__ __forceinline__ float bits2f(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t f2bits(float f) { return __float_as_uint(f); }

// ---- storage types ---------------------------------------------------------
struct F16 {
    using storage = uint16_t;
    static constexpr DType dt = kF16;
    __device__ __forceinline__ static float load(storage s) {
        return (float)__builtin_bit_cast(_Float16, s);
    }
    __device__ __forceinline__ static storage store(float v) {
        // Keep the fp32 value opaque: otherwise the backend folds (fp16)(a * b)
        // into v_fma_mixlo_f16 a, b, +0, which turns a -0 product into +0 and
        // rounds the product once instead of fp32-then-fp16.
        asm("" : "+v"(v));
        return __builtin_bit_cast(uint16_t, (_Float16)v);   // v_cvt_f16_f32: RNE, subnormals kept
    }
    __device__ __forceinline__ static float round(float v) { return load(store(v)); }
};

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

struct BF16 {
    using storage = uint16_t;
    static constexpr DType dt = kBF16;
    __device__ __forceinline__ static float load(storage s) { return bits2f((uint32_t)s << 16); }
    __device__ __forceinline__ static storage store(float v) {
        return __builtin_bit_cast(uint16_t, (__bf16)v);   // v_cvt_pk_bf16_f32: RNE, subnormals kept
    }
    // v_cvt_pk_bf16_f32 d, 0, v: the high half holds R(v), the low half R(0) = 0,
    // so d is already the float R(v) -- one instruction, no unpacking
    __device__ __forceinline__ static float round(float v) {
        return __builtin_bit_cast(float, __builtin_convertvector((f32x2_t){0.0f, v}, bf16x2_t));
    }
};

struct F32 {
    using storage = float;
    static constexpr DType dt = kF32;
    __device__ __forceinline__ static float load(storage s) { return s; }
    __device__ __forceinline__ static storage store(float v) { return v; }
    __device__ __forceinline__ static float round(float v) { return v; }
};

// Round two floats to T.  (For bf16 one v_cvt_pk_bf16_f32 per value beats one
// per pair: the pair would need two instructions to unpack.)
template <class T>
__device__ __forceinline__ void round2(float a, float b, float& ra, float& rb) {
    ra = T::round(a);
    rb = T::round(b);
}

// ---- binade exponent and the rounded-log2 exponent ------------------------
// True exponent e of a positive finite float (2^e <= a < 2^(e+1)), subnormals included.
__device__ __forceinline__ int binade(float a) { return __builtin_amdgcn_frexp_expf(a) - 1; }

// Where log2_exponent reads its per-binade thresholds: the __constant__ tables
// of log2_tables.h (ConstLog2), or copies of T's two tables that a kernel keeps
// in LDS (LdsLog2: entry e - EMIN of T), which saves a dependent global load.
struct ConstLog2 {};
struct LdsLog2 {
    const float* floor_thr;
    const float* round_thr;
};

// floor(R_T(log2 a)) (round_mode 0) or rint(R_T(log2 a)) (round_mode 1) for a
// positive finite T value a, from the per-binade thresholds in log2_tables.h.
template <class T, class Tab = ConstLog2>
__device__ __forceinline__ float log2_exponent(float a, int round_mode, Tab tab = Tab()) {
    int e = binade(a);
    float thr;
    if constexpr (std::is_same<Tab, LdsLog2>::value) {
        const int i = e - (T::dt == kF16 ? HBQ_L2T_F16_EMIN : T::dt == kBF16 ? HBQ_L2T_BF16_EMIN : HBQ_L2T_F32_EMIN);
        thr = round_mode ? tab.round_thr[i] : tab.floor_thr[i];
    } else if (T::dt == kF16) {
        int i = e - HBQ_L2T_F16_EMIN;
        thr = round_mode ? kLog2RoundF16[i] : kLog2FloorF16[i];
    } else if (T::dt == kBF16) {
        int i = e - HBQ_L2T_BF16_EMIN;
        thr = round_mode ? kLog2RoundBF16[i] : kLog2FloorBF16[i];
    } else {
        int i = e - HBQ_L2T_F32_EMIN;
        thr = round_mode ? kLog2RoundF32[i] : kLog2FloorF32[i];
    }
    return (float)(e + (a >= thr ? 1 : 0));
}

__device__ __forceinline__ float pow2f(int e) { return __builtin_amdgcn_ldexpf(1.0f, e); }

// ---- scale quantizer: fp_quant with rounding 0.5 or ceil (src/quantizer.py:259-328),
// applied after the clip to [min, max] of the scale format (src/quantizer.py:735-739).
// Inputs are T values; the result is a T value.
struct ScaleFmt {
    float lo, hi;        // clip bounds
    float emin, emax;    // exponent range of the scale format
    float thr, minn;     // subnormal threshold and min normal of the scale format
    float mmax, mshift;
    int allow_sub, use_ceil;
    int e4m3;            // E4M3 saturates at +-448
};

template <class T, class Tab = ConstLog2>
__device__ __forceinline__ float scale_quant(float s, const ScaleFmt& f, Tab tab = Tab()) {
    // clip (NaN passes through)
    s = s < f.lo ? f.lo : (s > f.hi ? f.hi : s);
    s = T::round(s);
    if (s != s) return s;
    float a = fabsf(s);
    bool is_zero = (s == 0.f);
    bool promote = (a < f.minn) && (a >= f.thr);
    bool sub = f.allow_sub && (a < f.thr) && !is_zero;
    bool under = !f.allow_sub && (a < f.thr) && !is_zero;
    float fe = a == __builtin_inff() ? a : log2_exponent<T>(is_zero ? 1.f : a, 0, tab);
    float e = fe < f.emin ? f.emin : (fe > f.emax ? f.emax : fe);
    // division by a power of two = multiplication by its exact reciprocal
    float rp2 = pow2f(-(int)e);
    float sg = s > 0.f ? 1.f : (s < 0.f ? -1.f : 0.f);
    float mant = sub ? T::round(T::round(s * rp2) * f.mshift)
                     : T::round(T::round(T::round(s * rp2) - sg) * f.mshift);
    float mr = f.use_ceil ? ceilf(fabsf(mant)) : floorf(T::round(fabsf(mant) + 0.5f));
    bool overflow = (mr > f.mmax) && (e != f.emax);
    if (mr > f.mmax) mr = f.mmax;
    if (is_zero || under || overflow || promote) mr = 0.f;
    if (overflow) e = e + 1.f;
    float sm = sg * mr;
    float p2b = T::round(pow2f((int)e));
    const float rshift = 1.0f / f.mshift;   // exact: mshift is a power of two
    float q = sub ? T::round(T::round(sm * rshift) * p2b)
                  : T::round(T::round(T::round(sm * rshift) + sg) * p2b);
    if (is_zero || under) q = 0.f;
    if (f.e4m3) q = q > 448.f ? 448.f : (q < -448.f ? -448.f : q);
    return q;
}

// E5M3 scale quantization of a positive normal T value s in [2^-14, 61440]
// (the L1 scale after its clip): rounding the fp32 mantissa to 3 bits half-up
// (or up, with use_ceil) is the reference's floor(R_T(|m| + 0.5)) / ceil(|m|)
// with the carry into the next binade.  With ceil, values whose R_T-rounded
// log2 already reaches the next binade take 1.125 * 2^(e+1) as in the reference.
template <class T>
__device__ __forceinline__ float e5m3_scale(float s, int use_ceil) {
    const uint32_t b = f2bits(s);
    if (!use_ceil) return bits2f((b + 0x80000u) & 0xfff00000u);
    const float q = bits2f((b + 0xfffffu) & 0xfff00000u);
    const int e = binade(s);
    const bool quirk = log2_exponent<T>(s, 0) > (float)e;
    return quirk ? 1.125f * pow2f(e + 1) : q;
}

// ---- element quantizer for E2Mm (src/quantizer.py:202-255, allow_subnormal=True).
// u is a T value.  Returns the quantized element value (in T) and its code
// [sign | exponent field (2 bits) | mantissa (m bits)], exponent field 0 for
// subnormals.  The exponent is taken from the binade: where the reference's
// floor(R_T(log2 u)) is one larger (u a few ulps below 2^(e+1)) both routes
// yield the same value, which the exhaustive element tests confirm.
//
// Two mantissa roundings, as the reference has two forms of this function:
//   fused = false: the eager op sequence; the Python scalar 0.5004 is rounded to
//     T and so is the sum, k = floor(R_T(|m| + R_T(0.5004)));
//   fused = true: the torch.compile'd function that GLOBAL_FP_QUANT_CACHE serves
//     (src/quantizer.py:38-63, HBQQuantizer's default use_quant_kernel=True): the
//     fused kernel computes in fp32, k = floor(f32(|m| + f32(0.5004))).
// |m| is exact in fp32 on both routes.  For fp32 tensors the two coincide.
template <class T, int M>
__device__ __forceinline__ float elem_quant(float u, uint32_t& code, bool fused = false) {
    constexpr float kShift = (float)(1 << M);
    constexpr float kInvShift = 1.0f / (float)(1 << M);
    constexpr float kMmax = (float)((1 << M) - 1);
    constexpr float kThr = 1.0f - 0.5f / (float)(1 << M);   // min_norm - 2^-(m+1)
    // T(0.5004): the scalar is rounded to T before the add
    const float rnd_eager = (T::dt == kF16) ? 0.50048828125f : (T::dt == kBF16 ? 0.5f : 0.5004f);
    const bool f32_sum = fused || T::dt == kF32;
    const float rnd = f32_sum ? 0.5004f : rnd_eager;
    float a = fabsf(u);
    uint32_t sbit = (f2bits(u) >> 31) << (M + 2);
    float q;
    if (a < kThr) {
        const float sum = a * kShift + rnd;   // a * 2^M is exact: one fp32 rounding
        float k = floorf(f32_sum ? sum : T::round(sum));
        if (k > kMmax) k = 0.f;   // rounds up into the normal range: the reference zeroes it
        q = (u == 0.f) ? 0.f : copysignf(k * kInvShift, u);
        code = (u == 0.f) ? 0u : (sbit | (uint32_t)k);
    } else if (a < 1.0f) {
        q = copysignf(1.0f, u);
        code = sbit | (1u << M);
    } else {
        int e = a >= 4.0f ? 2 : binade(a);     // also covers +inf (saturates below)
        float m = (a * pow2f(-e) - 1.0f) * kShift;
        const float sum = m + rnd;
        float k = floorf(f32_sum ? sum : T::round(sum));
        if (k > kMmax) {
            if (e < 2) { k = 0.f; e += 1; } else { k = kMmax; }
        }
        q = copysignf((1.0f + k * kInvShift) * pow2f(e), u);
        code = sbit | ((uint32_t)(e + 1) << M) | (uint32_t)k;
    }
    return q;
}

// R_T(x / s) for a scale s with reciprocal rs = 1/s (correctly rounded).
// For fp16/bf16, x * rs lies within 2^-23 (relative) of x / s and no quotient
// of a T value by an E5M3 scale or an L2 factor lies that close to a rounding
// boundary of T in the normal range (checked exhaustively by the CPU tests), so
// rounding the product gives R_T(x / s).  Quotients in T's subnormal range can
// be exact ties, so they take the IEEE division.
template <class T>
__device__ __forceinline__ float div_T(float x, float s, float rs) {
    if (T::dt == kF32) return x / s;
    float q = x * rs;
    const float tiny = (T::dt == kF16) ? 6.103515625e-05f : 1.17549435e-38f;
    if (fabsf(q) < tiny) return T::round(x / s);
    return T::round(q);
}

// wave-level helpers -------------------------------------------------------
// Max of 32-bit patterns across groups of G lanes (G a power of two <= 64).
template <int G>
__device__ __forceinline__ uint32_t group_max_u32(uint32_t v) {
#pragma unroll
    for (int off = 1; off < G; off <<= 1) {
        uint32_t o = (uint32_t)__shfl_xor((int)v, off, 64);
        v = v > o ? v : o;
    }
    return v;
}

}  // namespace hbq
