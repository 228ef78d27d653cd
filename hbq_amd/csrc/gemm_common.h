// Shared pieces of the block-quant GEMM kernels: operand types, the psum
// quantizers of blockquant_ext (blockquant_ext_src/gemm.cu:677-745, 1145-1251)
// and the per-K-group epilogue that folds an fp32 MFMA partial into the fp16
// accumulators (gemm.cu:354-377, 810-887, 1198-1277):
//   grouped : H = R16(H + R16(P))
//   mxint8  : per (row, GN columns) s = 2^(ilogb(max|P|) - 6), Q = clamp(rne(P/s), +-127) * s,
//             H = R16(H + R16(Q))
//   mxfp8   : same with E3M4 quantize-dequantize and s = 2^(ilogb(max|P|) - 3)
//
// Register layout (both kernels swap the MFMA operands, D = B^T A^T): a
// v_mfma_f32_32x32x16_f16 accumulator of a 32x32 block holds, in lane l,
// output row m = l % 32 and the 16 columns n = 8*(r/4) + 4*(l/32) + r%4 of
// register r; the other 16 columns of that row sit in lane l ^ 32.
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

namespace hbq_gemm {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float f2_t __attribute__((ext_vector_type(2)));

enum Mode : int { kGrouped = 0, kInt8 = 1, kFp8 = 2, kFp32 = 3, kPartial = 4 };

// ---- psum quantizers -------------------------------------------------------
__device__ __forceinline__ float int8_qdq(float p, float s, float inv) {
    float v = p * inv;
    if (v != v) return v;
    float q = rintf(v);
    q = q > 127.f ? 127.f : (q < -127.f ? -127.f : q);
    return q * s;
}

__device__ __forceinline__ float e3m4_qdq(float x, float scale) {
    float sgn = copysignf(1.f, x);
    float a = fabsf(x);
    if (a == 0.f) return copysignf(0.f, x);
    float y = a / scale;
    if (!isfinite(y)) {
        if (isnan(y)) return copysignf(__builtin_nanf(""), x);
        return sgn * 15.5f * scale;
    }
    if (y < 0.5f * 0.015625f) return 0.f;
    if (y >= 0.25f) {
        int e = __builtin_amdgcn_frexp_expf(y) - 1;   // exact floor(log2 y)
        e = e < -2 ? -2 : (e > 3 ? 3 : e);
        float p2 = __builtin_amdgcn_ldexpf(1.f, e);
        float frac = y / p2 - 1.f;
        float mant = rintf(frac * 16.f);
        if (mant >= 16.f) {
            mant = 0.f;
            ++e;
            if (e > 3) { e = 3; mant = 15.f; }
            p2 = __builtin_amdgcn_ldexpf(1.f, e);
        }
        float yq = (1.f + mant * (1.f / 16.f)) * p2;
        if (yq > 15.5f) yq = 15.5f;
        return sgn * yq * scale;
    }
    float mant = rintf(y * 64.f);
    if (mant <= 0.f) return 0.f;
    if (mant >= 16.f) return sgn * 0.25f * scale;
    float yq = (mant * (1.f / 16.f)) * 0.25f;
    return sgn * yq * scale;
}

// power-of-two psum scale 2^(ilogb(mx) - shift); 1 for an all-zero group; inf for an inf max
__device__ __forceinline__ float psum_scale(float mx, int shift) {
    if (!(mx > 0.f)) return 1.f;
    if (mx == __builtin_inff()) return __builtin_inff();
    return __builtin_amdgcn_ldexpf(1.f, __builtin_amdgcn_frexp_expf(mx) - 1 - shift);
}

// R16 of two fp32 values in one v_cvt_pk_f16_f32 (round to nearest even)
__device__ __forceinline__ h2_t cvt2(float a, float b) {
    h2_t q = __builtin_convertvector((f2_t){a, b}, h2_t);
    asm("" : "+v"(q));
    return q;
}

// max with the partner lane l ^ 32.  v_permlane32_swap exchanges the upper
// 32 lanes of its first operand with the lower 32 lanes of its second; with
// both operands holding v, the two results together hold v of lane l ^ 32 in
// every lane, whichever way the halves are assigned.  (Inline asm: the
// compiler treats the two results of the builtin as equal when its operands
// are, and drops one of them.)
__device__ __forceinline__ float xlane32_max(float v) {
    float a = v, b = v;
    // s_nop: the VALU-write -> permlane-read hazard the compiler inserts for the builtin
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    return fmaxf(v, fmaxf(a, b));
}

// R16(t0 - M0) and R16(t1 - M1) packed in one register.  The differences are exact
// in fp32 (t and M lie within a factor of 2), so two v_sub_f32 and one
// v_cvt_pk_f16_f32 round each once.  (A v_fma_mix per value does the same in one
// instruction, but issues at half the rate of a conversion and a quarter of a
// subtraction; the barriers keep the compiler from forming it.)
__device__ __forceinline__ h2_t sub_pair2(float t0, float M0, float t1, float M1) {
    float d0 = t0 - M0, d1 = t1 - M1;
    asm("" : "+v"(d0), "+v"(d1));
    return cvt2(d0, d1);
}
__device__ __forceinline__ h2_t sub_pair(float t0, float t1, float M) { return sub_pair2(t0, M, t1, M); }

__device__ __forceinline__ bool wave_any(bool p) { return __builtin_amdgcn_ballot_w64(p) != 0; }

// mxfp8 (E3M4, s = 2^(ilogb(mx) - 3)) of one partial P with the group's subnormal
// magic constant msub: the E3M4 grid step is 2^(ilogb P - 4) for |P| >= s / 4 and
// s / 64 below, so M = 1.5 * 2^23 * step = max(1.5 * 2^(ilogb P + 19), msub) (as
// float bit patterns, which order like the positive floats) and (P + M) - M is P
// rounded to the grid, ties to even as the reference's nearbyintf.
__device__ __forceinline__ float e3m4_magic(float P, uint32_t msub) {
    const uint32_t mn = (__builtin_bit_cast(uint32_t, P) & 0x7f800000u) + (19u << 23) + 0x400000u;
    return __builtin_bit_cast(float, mn > msub ? mn : msub);
}

// Fold the 16 fp32 partials of one 32x32 block into the fp16 accumulators H
// (8 packed pairs; pair p holds registers 2p and 2p + 1, adjacent columns).
//
// mxint8: with the group max mx normal, s = 2^(ilogb(mx) - 6), |P| / s < 128,
// and rne(P / s) * s = (P + M) - M with M = 1.5 * 2^23 * s: the add rounds P
// to the nearest (even) multiple of ulp(M) = s and the subtraction is exact.
// (fp16 products bound |P| by 2^39 and nonzero |P| below by 2^-48.)  A pair's
// two exact differences round to fp16 in one v_cvt_pk_f16_f32.  NaN partials stay
// NaN, as in the reference.  Only a group whose max has a mantissa of at least
// 1 + 127/128 (mx / s >= 127.5) can round to +-128 s; when a lane of the wave
// holds such a group the block also clamps, on the fp16 values: R16 is
// monotone and only +-128 s exceeds 127 s, so clamping R16(q) to +-R16(127 s)
// gives R16(clamp(q)), and v_pk_minimum3/maximum3 propagate NaN.  An all-zero
// group (mx = 0) gets M = 1.5 * 2^-110 from the same bit arithmetic, which
// turns every +-0 into +0 (the sign of a zero addend cannot change an
// accumulator that starts at +0 and only adds fp16 values).  The magic
// constants stay normal floats for a max in [2^-100, 2^110); with fp16 operands
// a nonzero partial is at least 2^-48 (a multiple of the smallest product) and a
// finite one below 2^39, so only an infinite max (every output NaN, as
// P / inf * inf) leaves that range: when a lane holds one, the whole wave takes
// the exact formula.  The branches depend on wave-wide ballots, so they are
// scalar branches.
template <int MODE, int GN>
__device__ __forceinline__ void fold_block_impl(const f16v& acc, h2_t* H) {
    if constexpr (MODE == kGrouped) {
#pragma unroll
        for (int p = 0; p < 8; ++p) H[p] = H[p] + cvt2(acc[2 * p], acc[2 * p + 1]);
    } else {
        constexpr int RPG = GN >= 8 ? GN / 2 : 4;     // registers of one column group in this lane
        constexpr int NG = 16 / RPG;
        float mxg[NG];
        bool special = false, top = false;
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            float mx = 0.f;
#pragma unroll
            for (int r = g * RPG; r < (g + 1) * RPG; ++r) mx = fmaxf(mx, fabsf(acc[r]));
            if constexpr (GN >= 8) mx = xlane32_max(mx);
            mxg[g] = mx;
            special |= mx >= 0x1p110f;   // a nonzero max is at least 2^-48 (fp16 operands)
            top |= (__builtin_bit_cast(uint32_t, mx) & 0x7fffffu) >= 0x7f0000u;
        }
        if constexpr (MODE == kInt8) {
            if (__builtin_expect(!wave_any(special), 1)) {
                float Mg[NG];
#pragma unroll
                for (int g = 0; g < NG; ++g)   // 1.5 * 2^23 * 2^(ilogb(mx) - 6)
                    Mg[g] = __builtin_bit_cast(
                        float, (__builtin_bit_cast(uint32_t, mxg[g]) & 0x7f800000u) + (17u << 23) + 0x400000u);
                if (__builtin_expect(!wave_any(top), 1)) {
                    // all 16 magic adds, then all 16 exact subtractions, then the 8 paired
                    // conversions: independent instructions back to back instead of one
                    // add-subtract-convert chain per pair (which also waits a cycle before
                    // each conversion); the barrier keeps the compiler from interleaving
                    // them again or forming v_fma_mix
                    float t[16];
#pragma unroll
                    for (int g = 0; g < NG; ++g)
#pragma unroll
                        for (int r = g * RPG; r < (g + 1) * RPG; ++r) t[r] = acc[r] + Mg[g];
#pragma unroll
                    for (int g = 0; g < NG; ++g)
#pragma unroll
                        for (int r = g * RPG; r < (g + 1) * RPG; ++r) t[r] = t[r] - Mg[g];
                    asm("" : "+v"(t[0]), "+v"(t[1]), "+v"(t[2]), "+v"(t[3]), "+v"(t[4]), "+v"(t[5]), "+v"(t[6]),
                        "+v"(t[7]), "+v"(t[8]), "+v"(t[9]), "+v"(t[10]), "+v"(t[11]), "+v"(t[12]), "+v"(t[13]),
                        "+v"(t[14]), "+v"(t[15]));
#pragma unroll
                    for (int p = 0; p < 8; ++p) H[p] = H[p] + cvt2(t[2 * p], t[2 * p + 1]);
                } else {
#pragma unroll
                    for (int g = 0; g < NG; ++g) {
                        const uint32_t mb = __builtin_bit_cast(uint32_t, mxg[g]);
                        const float s = mb != 0u ? __builtin_bit_cast(float, (mb & 0x7f800000u) - (6u << 23)) : 1.0f;
                        const _Float16 c = (_Float16)(127.0f * s);
                        const h2_t hi = (h2_t){c, c}, lo = -hi;
#pragma unroll
                        for (int r = g * RPG; r < (g + 1) * RPG; r += 2) {
                            const float t0 = acc[r] + Mg[g], t1 = acc[r + 1] + Mg[g];
                            const h2_t q = sub_pair(t0, t1, Mg[g]);
                            H[r / 2] = H[r / 2] + __builtin_elementwise_maximum(__builtin_elementwise_minimum(q, hi), lo);
                        }
                    }
                }
            } else {
                float q[16];
#pragma unroll
                for (int g = 0; g < NG; ++g) {
                    const float s = psum_scale(mxg[g], 6);
#pragma unroll
                    for (int r = g * RPG; r < (g + 1) * RPG; ++r) q[r] = int8_qdq(acc[r], s, 1.f / s);
                }
#pragma unroll
                for (int p = 0; p < 8; ++p) H[p] = H[p] + cvt2(q[2 * p], q[2 * p + 1]);
            }
        } else {
            // mxfp8: the fast path needs the group max below 2^100 (a nonzero max is at
            // least 2^-48), where the magic constants stay normal floats; a max with a mantissa of at least
            // 1 + 31/32 (mx / s >= 15.75) can round to 16 s, which the clamp to
            // R16(15.5 s) turns into the reference's 15.5 s
            bool special8 = false, top8 = false;
#pragma unroll
            for (int g = 0; g < NG; ++g) {
                special8 |= mxg[g] >= 0x1p100f;
                top8 |= (__builtin_bit_cast(uint32_t, mxg[g]) & 0x7fffffu) >= 0x7c0000u;
            }
            if (__builtin_expect(!wave_any(special8), 1)) {
                auto run = [&](auto clamp_tag) __attribute__((always_inline)) {
                    constexpr bool CLAMP = decltype(clamp_tag)::value;
#pragma unroll
                    for (int g = 0; g < NG; ++g) {
                        const uint32_t mb = __builtin_bit_cast(uint32_t, mxg[g]);
                        const uint32_t sb = (mb & 0x7f800000u) - (3u << 23);   // s (wraps for mx = 0, harmless)
                        const uint32_t msub = sb + (17u << 23) + 0x400000u;    // 1.5 * 2^23 * s / 64
#pragma unroll
                        for (int r = g * RPG; r < (g + 1) * RPG; r += 2) {
                            const float M0 = e3m4_magic(acc[r], msub), M1 = e3m4_magic(acc[r + 1], msub);
                            const float t0 = acc[r] + M0, t1 = acc[r + 1] + M1;
                            h2_t q = sub_pair2(t0, M0, t1, M1);
                            if constexpr (CLAMP) {
                                const _Float16 c =
                                    (_Float16)(15.5f * (mb != 0u ? __builtin_bit_cast(float, sb) : 1.0f));
                                const h2_t hi = (h2_t){c, c};
                                q = __builtin_elementwise_maximum(__builtin_elementwise_minimum(q, hi), -hi);
                            }
                            H[r / 2] = H[r / 2] + q;
                        }
                    }
                };
                if (__builtin_expect(!wave_any(top8), 1)) run(std::false_type{});
                else run(std::true_type{});
            } else {
                float q[16];
#pragma unroll
                for (int g = 0; g < NG; ++g) {
                    const float s = psum_scale(mxg[g], 3);
#pragma unroll
                    for (int r = g * RPG; r < (g + 1) * RPG; ++r) q[r] = e3m4_qdq(acc[r], s);
                }
#pragma unroll
                for (int p = 0; p < 8; ++p) H[p] = H[p] + cvt2(q[2 * p], q[2 * p + 1]);
            }
        }
    }
}

template <int MODE, int GN>
__device__ __forceinline__ void fold_block(const f16v& acc, h2_t* H) {
    fold_block_impl<MODE, GN>(acc, H);
    // H is final here: without this the compiler may defer the packed adds of a
    // psum group past the next K slice, keeping the 8 quantized pairs of every
    // block live across it (64 extra registers, spills)
    if constexpr (MODE != kGrouped) {
#pragma unroll
        for (int p = 0; p < 8; ++p) asm volatile("" : "+v"(H[p]));
    }
}

// fold_block over an R x C array of blocks with compile-time indices: the
// blocks' accumulators must stay in registers, and a loop the compiler declines
// to unroll (the exact paths make the body large) would index them dynamically
// and move them to scratch memory.
template <int MODE, int GN, int R, int C, int... B>
__device__ __forceinline__ void fold_all_impl(f16v (&acc)[R][C], h2_t (&H)[R][C][8], std::integer_sequence<int, B...>) {
    (fold_block<MODE, GN>(acc[B / C][B % C], H[B / C][B % C]), ...);
}
template <int MODE, int GN, int R, int C>
__device__ __forceinline__ void fold_all(f16v (&acc)[R][C], h2_t (&H)[R][C][8]) {
    fold_all_impl<MODE, GN>(acc, H, std::make_integer_sequence<int, R * C>{});
}

}  // namespace hbq_gemm
