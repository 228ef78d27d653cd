// Fused quantize-dequantize kernels for MXFP/NVFP and HBQ block formats on gfx950.
//
// Layout: the input is viewed as [rows, cols] with blocks of `block` elements
// along the last dimension (src/quantizer.py:67-146); a ragged last block is
// zero padded.  Each lane owns 16 consecutive elements of one block (two
// 16-byte loads for 16-bit types), so a block of B elements is handled by
// B/16 adjacent lanes of one wavefront.  One pass reads x once and writes the
// dequantized tensor, the element codes and the block scales.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "hbq_capi_internal.h"
#include "hbq_fast.h"
#include "mx_fast.h"
#include "quant_common.h"
#include "hbq_block.h"

namespace hbq {

// ---------------------------------------------------------------------------
// MXFP / NVFP  (MXFPQuantizer.get_shared_scale + q, src/quantizer.py:481-539)
// ---------------------------------------------------------------------------
template <class T, int M>
__global__ __launch_bounds__(kThreads) void mxfp_qdq_kernel(const typename T::storage* __restrict__ x,
                                                            typename T::storage* __restrict__ y,
                                                            typename T::storage* __restrict__ scales,
                                                            uint8_t* __restrict__ codes, int64_t cols, int block,
                                                            int lpb_log2, int64_t nblk_row, int64_t nb, MxParams p, bool ragged) {
    const Locate L = locate(lpb_log2, nblk_row, nb, block);
    float v[kV];
    load_lane<T>(x, L, cols, v, ragged);
    if (p.per_tensor) {
#pragma unroll
        for (int i = 0; i < kV; ++i) v[i] = T::round(v[i] / p.tscale);
    }
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < kV; ++i) {
        uint32_t b = f2bits(v[i]) & 0x7fffffffu;
        m = m > b ? m : b;
    }
    m = group_max_bits(m, 1 << lpb_log2);
    const float s = mx_shared_scale<T>(bits2f(m), p);
    const float rs = 1.0f / s;
    uint32_t c[kV];
#pragma unroll
    for (int i = 0; i < kV; ++i) {
        // a power-of-two scale divides exactly: rounding x * 2^-e is R_T(x / s)
        float yv = p.pot ? T::round(v[i] * rs) : div_T<T>(v[i], s, rs);
        float q = elem_quant<T, M>(yv, c[i], p.fused);
        float o = T::round(q * s);
        if (p.per_tensor) o = T::round(o * p.tscale);
        v[i] = o;
    }
    store_lane<T>(y, L, cols, v, ragged);
    if (L.valid) {
        store_codes<M>(codes, L.row, cols, L.c0, c, ragged);
        if (scales != nullptr && L.li == 0) scales[L.gb] = T::store(s);
    }
}

// ---------------------------------------------------------------------------
// HBQ  (HBQQuantizer.quant_scale + q, src/quantizer.py:735-859)
// ---------------------------------------------------------------------------
template <class T, int M, int L2B, int S>
__global__ __launch_bounds__(kThreads) void hbq_qdq_kernel(const typename T::storage* __restrict__ x,
                                                           typename T::storage* __restrict__ y,
                                                           typename T::storage* __restrict__ l1_out,
                                                           uint8_t* __restrict__ l2i_out, uint8_t* __restrict__ sch_out,
                                                           uint8_t* __restrict__ codes, int64_t cols, int block,
                                                           int lpb_log2, int64_t nblk_row, int64_t nb, HbqParams p, bool ragged) {
    constexpr int NSUBL = L2B <= kV ? kV / L2B : 1;   // sub-blocks held by one lane
    constexpr int LPS = L2B <= kV ? 1 : L2B / kV;     // lanes per sub-block
    const Locate L = locate(lpb_log2, nblk_row, nb, block);
    const int lpb = 1 << lpb_log2;
    const int lane = (int)(threadIdx.x & 63);

    float xv[kV];
    load_lane<T>(x, L, cols, xv, ragged);

    float out[kV];
    uint32_t cout[kV];
    float l1sel;
    int sstar;
    int jsel[NSUBL];
    hbq_block<T, M, L2B, S>(xv, L.li, lpb, lane, p, out, cout, l1sel, sstar, jsel);
    store_lane<T>(y, L, cols, out, ragged);
    if (!L.valid) return;
    store_codes<M>(codes, L.row, cols, L.c0, cout, ragged);
    if (L.li == 0) {
        if (l1_out) l1_out[L.gb] = T::store(l1sel);
        if (sch_out) sch_out[L.gb] = (uint8_t)sstar;
    }
    if (l2i_out) {
        const int nsub_blk = block / L2B;
        if (L2B <= kV) {
#pragma unroll
            for (int sb = 0; sb < NSUBL; ++sb) l2i_out[L.gb * nsub_blk + (L.li * kV) / L2B + sb] = (uint8_t)jsel[sb];
        } else if ((L.li % LPS) == 0) {
            l2i_out[L.gb * nsub_blk + (L.li * kV) / L2B] = (uint8_t)jsel[0];
        }
    }
}

// Elementwise fp_quant (src/quantizer.py:259-328), optionally after the clip
// to the format's range that quant_scale applies (src/quantizer.py:735-739).
template <class T>
__global__ __launch_bounds__(kThreads) void scale_quant_kernel(const typename T::storage* __restrict__ x,
                                                               typename T::storage* __restrict__ y, int64_t n,
                                                               ScaleFmt f) {
    int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    y[i] = T::store(scale_quant<T>(T::load(x[i]), f));
}

// Elementwise make_fp_quant (src/quantizer.py:187-257) for exhaustive checks of the element quantizer.
template <class T, int M>
__global__ __launch_bounds__(kThreads) void elem_quant_kernel(const typename T::storage* __restrict__ x,
                                                              typename T::storage* __restrict__ y,
                                                              uint8_t* __restrict__ codes, int64_t n, int fused) {
    int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    uint32_t c;
    float q = elem_quant<T, M>(T::load(x[i]), c, fused);
    y[i] = T::store(q);
    if (codes) codes[i] = (uint8_t)c;
}

}  // namespace hbq

// ===========================================================================
// Host launchers
// ===========================================================================
using namespace hbq;

namespace {

int ilog2_exact(int v) {
    int l = 0;
    while ((1 << l) < v) ++l;
    return (1 << l) == v ? l : -1;
}

double max_norm_h(int ebit, int mbit) {
    if (ebit == 4 && mbit == 3) return 448.0;
    int emax = (ebit == 5) ? 15 : (1 << (ebit - 1));
    return ldexp(1.0, emax) * (double)((1 << (mbit + 1)) - 1) / (double)(1 << mbit);
}
double min_norm_h(int ebit) { return ebit == 1 ? 1.0 : ldexp(1.0, 2 - (1 << (ebit - 1))); }
double min_subnorm_h(int ebit, int mbit) { return ldexp(1.0, 2 - (1 << (ebit - 1))) * ldexp(1.0, -mbit); }

float round_host(double v, int dt) {
    float f = (float)v;
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

int scale_fmt(ScaleFmt& f, int sc_ebit, int sc_mbit, int allow_sub, int use_ceil) {
    if (sc_ebit < 2 || sc_ebit > 5 || sc_mbit < 0 || sc_mbit > 7)
        return hbq_fail(HBQ_ERR_UNSUPPORTED, "scale format E%dM%d is not supported on the GPU path", sc_ebit, sc_mbit);
    int emin = 2 - (1 << (sc_ebit - 1));
    int emax = sc_ebit == 5 ? 15 : (1 << (sc_ebit - 1));
    f.lo = (float)(allow_sub ? min_subnorm_h(sc_ebit, sc_mbit) : min_norm_h(sc_ebit));
    f.hi = (float)max_norm_h(sc_ebit, sc_mbit);
    f.emin = (float)emin;
    f.emax = (float)emax;
    f.minn = (float)min_norm_h(sc_ebit);
    f.thr = (float)(min_norm_h(sc_ebit) - ldexp(1.0, -(sc_mbit + 1)) * ldexp(1.0, emin));
    f.mmax = (float)((1 << sc_mbit) - 1);
    f.mshift = (float)(1 << sc_mbit);
    f.allow_sub = allow_sub;
    f.use_ceil = use_ceil;
    f.e4m3 = (sc_ebit == 4 && sc_mbit == 3);
    return 0;
}

struct Geometry {
    int64_t nblk_row, nb;
    int lpb_log2;
    bool ragged;
    unsigned grid;
};

int geometry(Geometry& g, const void* x, const void* y, const void* codes, int64_t rows, int64_t cols, int block,
             int esize) {
    if (rows < 0 || cols < 0) return hbq_fail(HBQ_ERR_INVALID, "negative shape");
    int lb = ilog2_exact(block);
    if (lb < 4 || lb > 10)
        return hbq_fail(HBQ_ERR_UNSUPPORTED, "block_size %d is not supported on the GPU path (powers of two 16..1024)",
                        block);
    g.lpb_log2 = lb - 4;
    g.nblk_row = (cols + block - 1) / block;
    g.nb = rows * g.nblk_row;
    g.ragged = (cols % block) != 0 || ((uintptr_t)x % 16) != 0 || ((uintptr_t)y % 16) != 0 ||
               (codes != nullptr && ((uintptr_t)codes % 16) != 0) || ((cols * esize) % 16) != 0;
    int64_t lanes = g.nb << g.lpb_log2;
    int64_t grid = (lanes + kThreads - 1) / kThreads;
    if (grid > 0x7fffffff) return hbq_fail(HBQ_ERR_INVALID, "tensor too large");
    g.grid = (unsigned)grid;
    return 0;
}

template <class T, int M>
void launch_mx(const Geometry& g, const void* x, void* y, void* scales, void* codes, int64_t cols, int block,
               const MxParams& p, hipStream_t st) {
    using S = typename T::storage;
    hipLaunchKernelGGL((mxfp_qdq_kernel<T, M>), dim3(g.grid), dim3(kThreads), 0, st, (const S*)x, (S*)y, (S*)scales,
                       (uint8_t*)codes, cols, block, g.lpb_log2, g.nblk_row, g.nb, p, g.ragged);
}

template <class T>
int dispatch_mx_m(int mbit, const Geometry& g, const void* x, void* y, void* scales, void* codes, int64_t cols,
                  int block, const MxParams& p, hipStream_t st) {
    switch (mbit) {
        case 1: launch_mx<T, 1>(g, x, y, scales, codes, cols, block, p, st); return 0;
        case 2: launch_mx<T, 2>(g, x, y, scales, codes, cols, block, p, st); return 0;
        case 3: launch_mx<T, 3>(g, x, y, scales, codes, cols, block, p, st); return 0;
        case 5: launch_mx<T, 5>(g, x, y, scales, codes, cols, block, p, st); return 0;
        default: return hbq_fail(HBQ_ERR_UNSUPPORTED, "element format E2M%d is not supported on the GPU path", mbit);
    }
}

template <class T, int M, int L2B, int S>
void launch_hbq(const Geometry& g, const void* x, void* y, void* l1, void* l2i, void* sch, void* codes, int64_t cols,
                int block, const HbqParams& p, hipStream_t st) {
    using St = typename T::storage;
    hipLaunchKernelGGL((hbq_qdq_kernel<T, M, L2B, S>), dim3(g.grid), dim3(kThreads), 0, st, (const St*)x, (St*)y,
                       (St*)l1, (uint8_t*)l2i, (uint8_t*)sch, (uint8_t*)codes, cols, block, g.lpb_log2, g.nblk_row,
                       g.nb, p, g.ragged);
}

template <class T, int M, int S>
int dispatch_hbq_l2b(int l2b, const Geometry& g, const void* x, void* y, void* l1, void* l2i, void* sch, void* codes,
                     int64_t cols, int block, const HbqParams& p, hipStream_t st) {
    switch (l2b) {
        case 4: launch_hbq<T, M, 4, S>(g, x, y, l1, l2i, sch, codes, cols, block, p, st); return 0;
        case 8: launch_hbq<T, M, 8, S>(g, x, y, l1, l2i, sch, codes, cols, block, p, st); return 0;
        case 16: launch_hbq<T, M, 16, S>(g, x, y, l1, l2i, sch, codes, cols, block, p, st); return 0;
        case 32: launch_hbq<T, M, 32, S>(g, x, y, l1, l2i, sch, codes, cols, block, p, st); return 0;
        default:
            return hbq_fail(HBQ_ERR_UNSUPPORTED, "l2_block_size %d is not supported on the GPU path (4, 8, 16 or 32)",
                            l2b);
    }
}

template <class T>
int dispatch_hbq(int mbit, int S, int l2b, const Geometry& g, const void* x, void* y, void* l1, void* l2i, void* sch,
                 void* codes, int64_t cols, int block, const HbqParams& p, hipStream_t st) {
#define HBQ_CASE(MB, SS)                                                                             \
    if (mbit == MB && S == SS) return dispatch_hbq_l2b<T, MB, SS>(l2b, g, x, y, l1, l2i, sch, codes, cols, block, p, st);
    HBQ_CASE(1, 1) HBQ_CASE(1, 2) HBQ_CASE(2, 1) HBQ_CASE(2, 2) HBQ_CASE(3, 1) HBQ_CASE(3, 2)
#undef HBQ_CASE
    return hbq_fail(HBQ_ERR_UNSUPPORTED, "element format E2M%d is not supported by the HBQ GPU path", mbit);
}

}  // namespace

static int g_hbq_force_generic = 0;

// ---------------------------------------------------------------------------
// non-finite check of a GEMM output (the test of src/module.py:51-66 without a
// host synchronization): flag = 1 if any element has an all-ones exponent.
// rows x cols elements, row stride ld; VEC: every row start 16-byte aligned and
// cols * esize a multiple of 16 (16-byte loads), else one element per load.
// ---------------------------------------------------------------------------
template <bool VEC>
__global__ __launch_bounds__(kThreads) void nonfinite_kernel(const uint8_t* __restrict__ x, int64_t rows, int64_t cols,
                                                             int64_t ld, int esize, uint32_t em,
                                                             int* __restrict__ flag) {
    // em: the exponent fields of the elements of a 32-bit word (two 16-bit elements or one fp32)
    const uint32_t elo = esize == 4 ? em : (em & 0xffffu), ehi = esize == 4 ? 0u : (em & 0xffff0000u);
    auto bad_word = [&](uint32_t w) __attribute__((always_inline)) {
        return ((w & elo) == elo) | (esize != 4 && (w & ehi) == ehi);
    };
    bool bad = false;
    const int64_t per_row = VEC ? cols * esize / 16 : cols;   // units per row
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
        const uint8_t* row = x + r * ld * esize;
        for (int64_t c = (int64_t)blockIdx.x * kThreads + threadIdx.x; c < per_row; c += (int64_t)gridDim.x * kThreads) {
            if constexpr (VEC) {
                const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(row) + c);
                bad |= bad_word(v.x) | bad_word(v.y) | bad_word(v.z) | bad_word(v.w);
            } else {
                uint32_t w;
                if (esize == 4) w = *reinterpret_cast<const uint32_t*>(row + c * 4);
                else w = *reinterpret_cast<const uint16_t*>(row + c * 2);
                bad |= (w & elo) == elo;
            }
        }
    }
    if (bad) *flag = 1;
}

namespace hbq {

int hbq_l2_table(HbqParams& p, int& S, int l2_sc_bit, int l2_scheme, int dtype) {
    if (l2_sc_bit < 0 || l2_sc_bit > 3)
        return hbq_fail(HBQ_ERR_UNSUPPORTED, "l2_sc_bit %d not supported on the GPU path (0..3)", l2_sc_bit);
    p.J = 1 << l2_sc_bit;
    S = 1;
    // L2 candidate tables (src/quantizer.py:745-770), each entry rounded to T
    for (int r = 0; r < p.J; ++r) {
        double rr = r, b1 = 1 << l2_sc_bit, b2 = 1 << (l2_sc_bit + 1), b3 = 1 << (l2_sc_bit + 2);
        double fp = 1 + rr / b1, fp10 = 1 + rr / b2;
        double v;
        switch (l2_scheme) {
            case 0: v = ldexp(1.0, r); break;
            case 1: v = rr + 1; break;
            case 2: v = 1 + rr / 2; break;
            case 3: v = fp; break;
            case 4: v = 1 + (rr + 1) / b1; break;
            case 5: v = fp10; break;
            case 6: v = 1 + rr / b3; break;
            case 7: v = fp; S = 2; break;
            default: return hbq_fail(HBQ_ERR_INVALID, "Invalid L2 scheme code %d", l2_scheme);
        }
        p.l2[r][0] = round_host(v, dtype);
        p.l2[r][1] = round_host(l2_scheme == 7 ? fp10 : v, dtype);
        p.rl2[r][0] = 1.0f / p.l2[r][0];
        p.rl2[r][1] = 1.0f / p.l2[r][1];
    }
    return 0;
}

}  // namespace hbq

// ---------------------------------------------------------------------------
// scores of causal attention: s = R(R(s * scale) + bias) with bias 0 on and below
// the diagonal and -inf above it, the two elementwise ops of src/module.py:96-112
// (attn_weight = q @ k^T * scale_factor; attn_weight += attn_bias) in one pass.
// torch computes both in fp32 on the T values (the scalar as fp32) and rounds
// each result to T; so does this.  [mats, T, T], in place, 8 elements a thread.
// ---------------------------------------------------------------------------
template <class T>
__global__ __launch_bounds__(kThreads) void scale_causal_mask_kernel(typename T::storage* __restrict__ s, int64_t mats,
                                                                     int64_t Tn, float scale) {
    const int64_t per_row = Tn / 8;
    const int64_t total = mats * Tn * per_row;
    const int64_t u = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (u >= total) return;
    const int64_t row = u / per_row;
    const int64_t c0 = (u - row * per_row) * 8;
    const int64_t i = row % Tn;
    u32x4 v = *reinterpret_cast<const u32x4*>(s + row * Tn + c0);
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint16_t b = (uint16_t)(w[e / 2] >> (16 * (e % 2)));
        const float scaled = T::round(T::load(b) * scale);
        const float out = T::round(scaled + (c0 + e > i ? -__builtin_inff() : 0.0f));
        // torch's float -> bf16 conversion returns the canonical 0x7FC0 for every NaN
        // (inf - inf gives a negative NaN here); its float -> fp16 conversion keeps the sign
        const uint32_t o = (T::dt == kBF16 && out != out) ? 0x7FC0u : (uint32_t)T::store(out);
        w[e / 2] = (e % 2) ? ((w[e / 2] & 0xffffu) | (o << 16)) : ((w[e / 2] & 0xffff0000u) | o);
    }
    *reinterpret_cast<u32x4*>(s + row * Tn + c0) = (u32x4){w[0], w[1], w[2], w[3]};
}

// ---------------------------------------------------------------------------
// rotary embedding of q or k: y = R(R(x * cos) + R(rotate_half(x) * sin)),
// rotate_half(x) = cat(-x[d/2:], x[:d/2]), the three elementwise steps of the
// Llama attention in one pass, read from the projection's strided [b, t, h, d]
// view and written contiguous as [b, h, t, d].  Each step is torch's: fp32 on
// the T values, rounded to T (bf16 NaNs become torch's canonical 0x7FC0).
// cos / sin: [t, d] in T.  8 elements a thread.
// ---------------------------------------------------------------------------
template <class T>
__global__ __launch_bounds__(kThreads) void rope_kernel(const typename T::storage* __restrict__ x,
                                                        typename T::storage* __restrict__ y,
                                                        const typename T::storage* __restrict__ cs,
                                                        const typename T::storage* __restrict__ sn, int64_t B,
                                                        int64_t H, int64_t Tn, int64_t D, int64_t sb, int64_t st,
                                                        int64_t sh) {
    const int64_t per_row = D / 8;
    const int64_t u = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (u >= B * H * Tn * per_row) return;
    const int64_t r = u / per_row, i0 = (u - r * per_row) * 8;
    const int64_t t = r % Tn, r2 = r / Tn, h = r2 % H, bb = r2 / H;
    const int64_t half = D / 2;
    const bool lower = i0 < half;
    const typename T::storage* xr = x + bb * sb + t * st + h * sh;
    auto load8 = [](const typename T::storage* p, float* v) __attribute__((always_inline)) {
        const u32x4 q = *reinterpret_cast<const u32x4*>(p);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = T::load((typename T::storage)(w[e / 2] >> (16 * (e % 2))));
    };
    float xv[8], xp[8], c[8], s8[8];
    load8(xr + i0, xv);
    load8(xr + (lower ? i0 + half : i0 - half), xp);
    load8(cs + t * D + i0, c);
    load8(sn + t * D + i0, s8);
    uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float a = T::round(xv[e] * c[e]);
        const float rot = lower ? -xp[e] : xp[e];
        const float b = T::round(rot * s8[e]);
        const float out = T::round(a + b);
        const uint32_t o = (T::dt == kBF16 && out != out) ? 0x7FC0u : (uint32_t)T::store(out);
        w[e / 2] |= o << (16 * (e % 2));
    }
    *reinterpret_cast<u32x4*>(y + ((bb * H + h) * Tn + t) * D + i0) = (u32x4){w[0], w[1], w[2], w[3]};
}

// ---------------------------------------------------------------------------
// causal attention probabilities from raw scores, in one pass:
//   e = R(R(s * scale) + bias)    (bias -inf above the diagonal; src/module.py:96-112)
//   p = softmax(e) along the row  (src/module.py:113, torch.softmax in fp32, rounded to T)
// The softmax follows torch's persistent warp softmax step for step, so the bits are
// torch's: one wave (64 lanes) per row, lane l holding columns l + 64 it; the row max
// by a sequential "a > b ? a : b" over its elements, then a butterfly over the lanes
// with "a < b ? b : a"; sum += exp(e - max) in column order, butterfly-added; p =
// exp(e - max) / sum (a NaN row for sum == 0), rounded to T (bf16 NaNs 0x7FC0).
// [mats, t, t] with t = 64 ITER, in place allowed (a row is read before it is written).
// ---------------------------------------------------------------------------
template <class T, int ITER>
__global__ __launch_bounds__(kThreads) void causal_softmax_kernel(const typename T::storage* __restrict__ s,
                                                                  typename T::storage* p, int64_t rows,
                                                                  float scale) {
    constexpr int Tn = 64 * ITER;
    const int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    if (row >= rows) return;   // whole waves
    const int lane = threadIdx.x & 63;
    const int64_t i = row % Tn;
    const typename T::storage* src = s + row * Tn;
    // rows of 512 or more: 16-byte global loads and stores staged through this wave's LDS
    // row, from which each lane takes its columns lane + 64 it (the reduction order)
    constexpr bool STAGE = ITER >= 8;
    __shared__ __attribute__((aligned(16))) uint16_t rowbuf[STAGE ? kThreads / 64 : 1][STAGE ? Tn : 8];
    uint16_t* rb = rowbuf[STAGE ? (threadIdx.x >> 6) : 0];
    if constexpr (STAGE) {
#pragma unroll
        for (int q = 0; q < ITER / 8; ++q) {
            const int c8 = 8 * (lane + 64 * q);
            *reinterpret_cast<u32x4*>(rb + c8) = *reinterpret_cast<const u32x4*>(src + c8);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    float el[ITER];
#pragma unroll
    for (int it = 0; it < ITER; ++it) {
        const int c = lane + 64 * it;
        const float scaled = T::round(T::load(STAGE ? rb[c] : src[c]) * scale);
        el[it] = T::round(scaled + (c > i ? -__builtin_inff() : 0.0f));
    }
    float mx = el[0];
#pragma unroll
    for (int it = 0; it < ITER; ++it) mx = mx > el[it] ? mx : el[it];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float b = __shfl_xor(mx, off, 64);
        mx = mx < b ? b : mx;
    }
    float sum = 0.f;
#pragma unroll
    for (int it = 0; it < ITER; ++it) {
        el[it] = expf(el[it] - mx);
        sum += el[it];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum = sum + __shfl_xor(sum, off, 64);
    typename T::storage* dst = p + row * Tn;
#pragma unroll
    for (int it = 0; it < ITER; ++it) {
        const float v = sum == 0.f ? __builtin_nanf("") : el[it] / sum;
        const typename T::storage o = (T::dt == kBF16 && v != v) ? (typename T::storage)0x7FC0u : T::store(v);
        if constexpr (STAGE) rb[lane + 64 * it] = o;
        else dst[lane + 64 * it] = o;
    }
    if constexpr (STAGE) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int q = 0; q < ITER / 8; ++q) {
            const int c8 = 8 * (lane + 64 * q);
            *reinterpret_cast<u32x4*>(dst + c8) = *reinterpret_cast<const u32x4*>(rb + c8);
        }
    }
}

extern "C" {

// Test hook: 1 routes every HBQ and MXFP / NVFP call to the generic kernels (so both can be
// checked); 2 makes a call that the table kernel declines fail instead of falling back.
int hbq_set_generic_only(int on) {
    int old = g_hbq_force_generic;
    g_hbq_force_generic = on;
    return old;
}

int hbq_mxfp_qdq(const void* x, void* y, void* scales, void* codes, int64_t rows, int64_t cols, int dtype,
                 int block_size, int ebit, int mbit, int sc_ebit, int sc_mbit, int scale_allow_subnormal,
                 int use_round, int use_ceil, int per_tensor_scale, double tensor_scale, int compiled,
                 void* stream) {
    hbq_clear_error();
    if (dtype != kF16 && dtype != kBF16 && dtype != kF32) return hbq_fail(HBQ_ERR_INVALID, "bad dtype code %d", dtype);
    if (ebit != 2) return hbq_fail(HBQ_ERR_UNSUPPORTED, "element exponent bits %d not supported on the GPU path", ebit);
    if (x == nullptr || y == nullptr) return hbq_fail(HBQ_ERR_INVALID, "null input/output pointer");
    int esize = dtype == kF32 ? 4 : 2;
    Geometry g;
    if (int rc = geometry(g, x, y, codes, rows, cols, block_size, esize)) return rc;
    if (g.nb == 0) return 0;
    MxParams p{};
    p.pot = sc_mbit == 0;
    p.use_round = use_round;
    p.ele_emax = (float)(1 << (ebit - 1));
    if (p.pot) {
        if (sc_ebit < 2 || sc_ebit > 8) return hbq_fail(HBQ_ERR_UNSUPPORTED, "PoT scale exponent bits %d", sc_ebit);
        p.sc_emax = (float)((1 << (sc_ebit - 1)) - 1);
        p.sc_emin = (float)(2 - (1 << (sc_ebit - 1)));
        p.min_normal = dtype == kF32 ? 1.17549435e-38f : 6.103515625e-05f;
    } else {
        if (int rc = scale_fmt(p.sf, sc_ebit, sc_mbit, scale_allow_subnormal, use_ceil)) return rc;
        p.ele_maxnorm = round_host(max_norm_h(ebit, mbit), dtype);
    }
    p.per_tensor = per_tensor_scale;
    p.tscale = round_host(tensor_scale, dtype);
    p.fused = compiled != 0;
    hipStream_t st = (hipStream_t)stream;
    if (g_hbq_force_generic != 1) {
        const int fr = hbq_mx_fast_try(x, y, scales, codes, rows, cols, dtype, block_size, mbit, p, st);
        if (fr < 0) return -fr;
        if (fr == 1) return hbq_check_launch("hbq_mxfp_qdq");
        if (g_hbq_force_generic == 2) return hbq_fail(HBQ_ERR_UNSUPPORTED, "the table kernel declined this call");
    }
    int rc;
    if (dtype == kF16) rc = dispatch_mx_m<F16>(mbit, g, x, y, scales, codes, cols, block_size, p, st);
    else if (dtype == kBF16) rc = dispatch_mx_m<BF16>(mbit, g, x, y, scales, codes, cols, block_size, p, st);
    else rc = dispatch_mx_m<F32>(mbit, g, x, y, scales, codes, cols, block_size, p, st);
    if (rc) return rc;
    return hbq_check_launch("hbq_mxfp_qdq");
}

// argument checks and candidate tables shared by the HBQ entry points
static int hbq_setup(HbqParams& p, int& S, Geometry& g, const void* x, const void* y, const void* codes, int64_t rows,
                     int64_t cols, int dtype, int block_size, int ebit, int mbit, int sc_ebit, int sc_mbit,
                     int l2_block_size, int l2_sc_bit, int l2_scheme, int scale_allow_subnormal, int use_ceil) {
    if (dtype != kF16 && dtype != kBF16 && dtype != kF32) return hbq_fail(HBQ_ERR_INVALID, "bad dtype code %d", dtype);
    if (ebit != 2) return hbq_fail(HBQ_ERR_UNSUPPORTED, "element exponent bits %d not supported on the GPU path", ebit);
    if (x == nullptr || y == nullptr) return hbq_fail(HBQ_ERR_INVALID, "null input/output pointer");
    if (l2_block_size <= 0 || block_size % l2_block_size != 0)
        return hbq_fail(HBQ_ERR_INVALID, "block_size must be divisible by l2_block_size");
    if (l2_sc_bit < 0 || l2_sc_bit > 3)
        return hbq_fail(HBQ_ERR_UNSUPPORTED, "l2_sc_bit %d not supported on the GPU path (0..3)", l2_sc_bit);
    int esize = dtype == kF32 ? 4 : 2;
    if (int rc = geometry(g, x, y, codes, rows, cols, block_size, esize)) return rc;
    if (l2_block_size > block_size) return hbq_fail(HBQ_ERR_INVALID, "l2_block_size larger than block_size");
    S = 1;
    if (int rc = hbq_l2_table(p, S, l2_sc_bit, l2_scheme, dtype)) return rc;
    const int J = p.J;
    float elemax = round_host(max_norm_h(ebit, mbit), dtype);
    for (int s = 0; s < S; ++s) {
        float m = p.l2[0][s];
        for (int j = 1; j < J; ++j) m = p.l2[j][s] > m ? p.l2[j][s] : m;
        p.em[s] = round_host((double)elemax * (double)m, dtype);
    }
    return scale_fmt(p.sf, sc_ebit, sc_mbit, scale_allow_subnormal, use_ceil);
}

int hbq_hbq_qdq(const void* x, void* y, void* l1_scale, void* l2_index, void* scheme, void* codes, int64_t rows,
                int64_t cols, int dtype, int block_size, int ebit, int mbit, int sc_ebit, int sc_mbit,
                int l2_block_size, int l2_sc_bit, int l2_scheme, int scale_allow_subnormal, int use_ceil,
                int compiled, void* stream) {
    hbq_clear_error();
    HbqParams p{};
    int S = 1;
    Geometry g;
    if (int rc = hbq_setup(p, S, g, x, y, codes, rows, cols, dtype, block_size, ebit, mbit, sc_ebit, sc_mbit,
                           l2_block_size, l2_sc_bit, l2_scheme, scale_allow_subnormal, use_ceil))
        return rc;
    p.fused = compiled != 0;
    if (g.nb == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    if (g_hbq_force_generic != 1) {
        int fr = hbq_fast_try(x, y, l1_scale, l2_index, scheme, codes, rows, cols, dtype, block_size, mbit,
                              l2_block_size, l2_sc_bit, l2_scheme, p, st);
        if (fr < 0) return -fr;
        if (fr == 1) return hbq_check_launch("hbq_hbq_qdq");
        if (g_hbq_force_generic == 2) return hbq_fail(HBQ_ERR_UNSUPPORTED, "the table kernel declined this call");
    }
    int rc;
    if (dtype == kF16) rc = dispatch_hbq<F16>(mbit, S, l2_block_size, g, x, y, l1_scale, l2_index, scheme, codes, cols, block_size, p, st);
    else if (dtype == kBF16) rc = dispatch_hbq<BF16>(mbit, S, l2_block_size, g, x, y, l1_scale, l2_index, scheme, codes, cols, block_size, p, st);
    else rc = dispatch_hbq<F32>(mbit, S, l2_block_size, g, x, y, l1_scale, l2_index, scheme, codes, cols, block_size, p, st);
    if (rc) return rc;
    return hbq_check_launch("hbq_hbq_qdq");
}

int hbq_hbq_qdq_causal(void* x, int64_t mats, int64_t t, int dtype, int block_size, int ebit, int mbit, int sc_ebit,
                       int sc_mbit, int l2_block_size, int l2_sc_bit, int l2_scheme, int scale_allow_subnormal,
                       int use_ceil, int compiled, void* stream) {
    hbq_clear_error();
    if (mats < 0 || t < 0) return hbq_fail(HBQ_ERR_INVALID, "negative size");
    if (t % 128 || block_size != 128)
        return hbq_fail(HBQ_ERR_UNSUPPORTED, "the causal quantizer takes block_size 128 and t %% 128 == 0");
    if (dtype != kF16 && dtype != kBF16) return hbq_fail(HBQ_ERR_UNSUPPORTED, "the causal quantizer takes fp16 / bf16");
    HbqParams p{};
    int S = 1;
    Geometry g;
    if (int rc = hbq_setup(p, S, g, x, x, nullptr, mats * t, t, dtype, block_size, ebit, mbit, sc_ebit, sc_mbit,
                           l2_block_size, l2_sc_bit, l2_scheme, scale_allow_subnormal, use_ceil))
        return rc;
    p.fused = compiled != 0;
    if (g.nb == 0) return 0;
    const int fr = g_hbq_force_generic == 1 ? 0
                                       : hbq_fast_try(x, x, nullptr, nullptr, nullptr, nullptr, mats * t, t, dtype,
                                                      block_size, mbit, l2_block_size, l2_sc_bit, l2_scheme, p,
                                                      (hipStream_t)stream, t);
    if (fr < 0) return -fr;
    if (fr == 0) return hbq_fail(HBQ_ERR_UNSUPPORTED, "configuration outside the table kernel's");
    return hbq_check_launch("hbq_hbq_qdq_causal");
}

// The HBQ quantizer on the output of the pass that produces it, computed in the
// quantizer's load step (the producer's output never written).
static int hbq_src_qdq(const FastSrc& src, void* y, int64_t rows, int64_t cols, int dtype, int block_size, int ebit,
                       int mbit, int sc_ebit, int sc_mbit, int l2_block_size, int l2_sc_bit, int l2_scheme,
                       int scale_allow_subnormal, int use_ceil, int compiled, void* stream, const char* name) {
    hbq_clear_error();
    if (rows < 0 || cols < 0) return hbq_fail(HBQ_ERR_INVALID, "negative size");
    if (dtype != kF16 && dtype != kBF16) return hbq_fail(HBQ_ERR_UNSUPPORTED, "%s takes fp16 / bf16", name);
    if (rows == 0 || cols == 0) return 0;
    if (!src.a || !src.b || !y || (src.kind == kSrcRms && !src.rs)) return hbq_fail(HBQ_ERR_INVALID, "null pointer");
    HbqParams p{};
    int S = 1;
    Geometry g;
    if (int rc = hbq_setup(p, S, g, src.a, y, nullptr, rows, cols, dtype, block_size, ebit, mbit, sc_ebit, sc_mbit,
                           l2_block_size, l2_sc_bit, l2_scheme, scale_allow_subnormal, use_ceil))
        return rc;
    p.fused = compiled != 0;
    if (g.nb == 0) return 0;
    const int fr = hbq_fast_try_src(src, y, rows, cols, dtype, block_size, mbit, l2_block_size, l2_sc_bit, l2_scheme,
                                    p, (hipStream_t)stream);
    if (fr < 0) return -fr;
    if (fr == 0)
        return hbq_fail(HBQ_ERR_UNSUPPORTED, "%s: configuration outside the fused kernels (E2M2 elements, one "
                        "L2 scheme, block 128, 16-byte aligned rows)", name);
    return hbq_check_launch(name);
}

int hbq_rms_apply_hbq_qdq(const void* x, const float* rs, const void* w, void* y, int64_t rows, int64_t cols,
                          int dtype, int block_size, int ebit, int mbit, int sc_ebit, int sc_mbit, int l2_block_size,
                          int l2_sc_bit, int l2_scheme, int scale_allow_subnormal, int use_ceil, int compiled,
                          void* stream) {
    const FastSrc src{kSrcRms, (const uint16_t*)x, (const uint16_t*)w, rs};
    return hbq_src_qdq(src, y, rows, cols, dtype, block_size, ebit, mbit, sc_ebit, sc_mbit, l2_block_size, l2_sc_bit,
                       l2_scheme, scale_allow_subnormal, use_ceil, compiled, stream, "hbq_rms_apply_hbq_qdq");
}

int hbq_silu_mul_hbq_qdq(const void* g, const void* u, void* y, int64_t rows, int64_t cols, int dtype,
                         int block_size, int ebit, int mbit, int sc_ebit, int sc_mbit, int l2_block_size,
                         int l2_sc_bit, int l2_scheme, int scale_allow_subnormal, int use_ceil, int compiled,
                         void* stream) {
    const FastSrc src{kSrcSilu, (const uint16_t*)g, (const uint16_t*)u, nullptr};
    return hbq_src_qdq(src, y, rows, cols, dtype, block_size, ebit, mbit, sc_ebit, sc_mbit, l2_block_size, l2_sc_bit,
                       l2_scheme, scale_allow_subnormal, use_ceil, compiled, stream, "hbq_silu_mul_hbq_qdq");
}

int hbq_scale_quant(const void* x, void* y, int64_t n, int dtype, int ebit, int mbit, int allow_subnormal,
                    int use_ceil, int clip, void* stream) {
    hbq_clear_error();
    if (n < 0 || x == nullptr || y == nullptr) return hbq_fail(HBQ_ERR_INVALID, "bad arguments");
    ScaleFmt f;
    if (int rc = scale_fmt(f, ebit, mbit, allow_subnormal, use_ceil)) return rc;
    if (!clip) {
        f.lo = -__builtin_inff();
        f.hi = __builtin_inff();
    }
    if (n == 0) return 0;
    int64_t grid = (n + kThreads - 1) / kThreads;
    if (grid > 0x7fffffff) return hbq_fail(HBQ_ERR_INVALID, "tensor too large");
    hipStream_t st = (hipStream_t)stream;
    if (dtype == kF16)
        hipLaunchKernelGGL(scale_quant_kernel<F16>, dim3((unsigned)grid), dim3(kThreads), 0, st, (const uint16_t*)x,
                           (uint16_t*)y, n, f);
    else if (dtype == kBF16)
        hipLaunchKernelGGL(scale_quant_kernel<BF16>, dim3((unsigned)grid), dim3(kThreads), 0, st, (const uint16_t*)x,
                           (uint16_t*)y, n, f);
    else if (dtype == kF32)
        hipLaunchKernelGGL(scale_quant_kernel<F32>, dim3((unsigned)grid), dim3(kThreads), 0, st, (const float*)x,
                           (float*)y, n, f);
    else return hbq_fail(HBQ_ERR_INVALID, "bad dtype code %d", dtype);
    return hbq_check_launch("hbq_scale_quant");
}

int hbq_elem_quant(const void* x, void* y, void* codes, int64_t n, int dtype, int ebit, int mbit, int compiled,
                   void* stream) {
    hbq_clear_error();
    if (ebit != 2) return hbq_fail(HBQ_ERR_UNSUPPORTED, "element exponent bits %d not supported on the GPU path", ebit);
    if (n < 0 || x == nullptr || y == nullptr) return hbq_fail(HBQ_ERR_INVALID, "bad arguments");
    if (n == 0) return 0;
    int64_t grid = (n + kThreads - 1) / kThreads;
    if (grid > 0x7fffffff) return hbq_fail(HBQ_ERR_INVALID, "tensor too large");
    hipStream_t st = (hipStream_t)stream;
#define ELEM_CASE(TT, MB)                                                                                          \
    hipLaunchKernelGGL((elem_quant_kernel<TT, MB>), dim3((unsigned)grid), dim3(kThreads), 0, st,                   \
                       (const TT::storage*)x, (TT::storage*)y, (uint8_t*)codes, n, compiled != 0)
#define ELEM_M(TT)                                                                                                 \
    switch (mbit) {                                                                                                \
        case 1: ELEM_CASE(TT, 1); break;                                                                           \
        case 2: ELEM_CASE(TT, 2); break;                                                                           \
        case 3: ELEM_CASE(TT, 3); break;                                                                           \
        case 5: ELEM_CASE(TT, 5); break;                                                                           \
        default: return hbq_fail(HBQ_ERR_UNSUPPORTED, "element format E2M%d not supported", mbit);               \
    }
    if (dtype == kF16) { ELEM_M(F16) }
    else if (dtype == kBF16) { ELEM_M(BF16) }
    else if (dtype == kF32) { ELEM_M(F32) }
    else return hbq_fail(HBQ_ERR_INVALID, "bad dtype code %d", dtype);
#undef ELEM_M
#undef ELEM_CASE
    return hbq_check_launch("hbq_elem_quant");
}

int hbq_scale_causal_mask(void* s, int64_t mats, int64_t t, double scale, int dtype, void* stream) {
    hbq_clear_error();
    if (dtype != kF16 && dtype != kBF16) return hbq_fail(HBQ_ERR_UNSUPPORTED, "scores must be fp16 or bf16");
    if (mats < 0 || t < 0) return hbq_fail(HBQ_ERR_INVALID, "negative size");
    if (t % 8) return hbq_fail(HBQ_ERR_UNSUPPORTED, "the sequence length must be a multiple of 8");
    if (mats == 0 || t == 0) return 0;
    if (s == nullptr || (uintptr_t)s % 16) return hbq_fail(HBQ_ERR_INVALID, "scores must be 16-byte aligned");
    const int64_t total = mats * t * (t / 8);
    const int64_t grid = (total + kThreads - 1) / kThreads;
    if (grid > 0x7fffffff) return hbq_fail(HBQ_ERR_INVALID, "tensor too large");
    if (dtype == kF16)
        hipLaunchKernelGGL(scale_causal_mask_kernel<F16>, dim3((unsigned)grid), dim3(kThreads), 0, (hipStream_t)stream,
                           (uint16_t*)s, mats, t, (float)scale);
    else
        hipLaunchKernelGGL(scale_causal_mask_kernel<BF16>, dim3((unsigned)grid), dim3(kThreads), 0,
                           (hipStream_t)stream, (uint16_t*)s, mats, t, (float)scale);
    return hbq_check_launch("hbq_scale_causal_mask");
}

int hbq_causal_softmax(const void* s, void* p, int64_t mats, int64_t t, double scale, int dtype, void* stream) {
    hbq_clear_error();
    if (dtype != kF16 && dtype != kBF16) return hbq_fail(HBQ_ERR_UNSUPPORTED, "scores must be fp16 or bf16");
    if (mats < 0) return hbq_fail(HBQ_ERR_INVALID, "negative size");
    if (t != 64 && t != 128 && t != 256 && t != 512 && t != 1024 && t != 2048)
        return hbq_fail(HBQ_ERR_UNSUPPORTED, "the fused causal softmax takes t = 64, 128, ..., 2048");
    if (mats == 0) return 0;
    if (!s || !p) return hbq_fail(HBQ_ERR_INVALID, "null pointer");
    if (((uintptr_t)s | (uintptr_t)p) % 16) return hbq_fail(HBQ_ERR_INVALID, "scores must be 16-byte aligned");
    const int64_t rows = mats * t;
    const int64_t grid = (rows + (kThreads / 64) - 1) / (kThreads / 64);
    if (grid > 0x7fffffff) return hbq_fail(HBQ_ERR_INVALID, "tensor too large");
    hipStream_t st = (hipStream_t)stream;
    const float sc = (float)scale;
#define CSM(TT, IT)                                                                                        \
    hipLaunchKernelGGL((causal_softmax_kernel<TT, IT>), dim3((unsigned)grid), dim3(kThreads), 0, st,       \
                       (const uint16_t*)s, (uint16_t*)p, rows, sc)
#define CSM_T(TT)                                                                                          \
    switch (t) {                                                                                           \
        case 64: CSM(TT, 1); break;                                                                        \
        case 128: CSM(TT, 2); break;                                                                       \
        case 256: CSM(TT, 4); break;                                                                       \
        case 512: CSM(TT, 8); break;                                                                       \
        case 1024: CSM(TT, 16); break;                                                                     \
        default: CSM(TT, 32); break;                                                                       \
    }
    if (dtype == kF16) { CSM_T(F16) } else { CSM_T(BF16) }
#undef CSM_T
#undef CSM
    return hbq_check_launch("hbq_causal_softmax");
}

int hbq_rope(const void* x, void* y, const void* cos, const void* sin, int64_t b, int64_t h, int64_t t, int64_t d,
             int64_t stride_b, int64_t stride_t, int64_t stride_h, int dtype, void* stream) {
    hbq_clear_error();
    if (dtype != kF16 && dtype != kBF16) return hbq_fail(HBQ_ERR_UNSUPPORTED, "rope takes fp16 or bf16");
    if (b < 0 || h < 0 || t < 0 || d < 0) return hbq_fail(HBQ_ERR_INVALID, "negative size");
    if (d % 16) return hbq_fail(HBQ_ERR_UNSUPPORTED, "rope needs head_dim %% 16 == 0");
    if (b == 0 || h == 0 || t == 0 || d == 0) return 0;
    if (!x || !y || !cos || !sin) return hbq_fail(HBQ_ERR_INVALID, "null pointer");
    if (((uintptr_t)x | (uintptr_t)y | (uintptr_t)cos | (uintptr_t)sin) % 16 || stride_b % 8 || stride_t % 8 ||
        stride_h % 8)
        return hbq_fail(HBQ_ERR_INVALID, "rope needs 16-byte aligned rows");
    const int64_t total = b * h * t * (d / 8);
    const int64_t grid = (total + kThreads - 1) / kThreads;
    if (grid > 0x7fffffff) return hbq_fail(HBQ_ERR_INVALID, "tensor too large");
    if (dtype == kF16)
        hipLaunchKernelGGL(rope_kernel<F16>, dim3((unsigned)grid), dim3(kThreads), 0, (hipStream_t)stream,
                           (const uint16_t*)x, (uint16_t*)y, (const uint16_t*)cos, (const uint16_t*)sin, b, h, t, d,
                           stride_b, stride_t, stride_h);
    else
        hipLaunchKernelGGL(rope_kernel<BF16>, dim3((unsigned)grid), dim3(kThreads), 0, (hipStream_t)stream,
                           (const uint16_t*)x, (uint16_t*)y, (const uint16_t*)cos, (const uint16_t*)sin, b, h, t, d,
                           stride_b, stride_t, stride_h);
    return hbq_check_launch("hbq_rope");
}

int hbq_flag_nonfinite(const void* x, int64_t rows, int64_t cols, int64_t ld, int dtype, int* flag, void* stream) {
    hbq_clear_error();
    if (dtype != kF16 && dtype != kBF16 && dtype != kF32) return hbq_fail(HBQ_ERR_INVALID, "bad dtype code %d", dtype);
    if (rows < 0 || cols < 0 || ld < cols || flag == nullptr) return hbq_fail(HBQ_ERR_INVALID, "bad arguments");
    if (rows == 0 || cols == 0) return 0;
    if (x == nullptr) return hbq_fail(HBQ_ERR_INVALID, "null tensor pointer");
    const int esize = dtype == kF32 ? 4 : 2;
    const uint32_t em = dtype == kF32 ? 0x7f800000u : (dtype == kF16 ? 0x7c007c00u : 0x7f807f80u);
    if (ld == cols) {   // contiguous: one long row
        cols *= rows;
        ld = cols;
        rows = 1;
    }
    const bool vec = (uintptr_t)x % 16 == 0 && (ld * esize) % 16 == 0 && (cols * esize) % 16 == 0;
    const int64_t per_row = vec ? cols * esize / 16 : cols;
    // about 4 units per thread, at most 2048 workgroups
    int64_t gx = (per_row + kThreads * 4 - 1) / (kThreads * 4);
    gx = gx > 2048 ? 2048 : gx;
    int64_t gy = 2048 / gx;
    gy = gy > rows ? rows : (gy > 65535 ? 65535 : gy);
    const dim3 grid((unsigned)gx, (unsigned)gy);
    if (vec)
        hipLaunchKernelGGL(nonfinite_kernel<true>, grid, dim3(kThreads), 0, (hipStream_t)stream,
                           (const uint8_t*)x, rows, cols, ld, esize, em, flag);
    else
        hipLaunchKernelGGL(nonfinite_kernel<false>, grid, dim3(kThreads), 0, (hipStream_t)stream,
                           (const uint8_t*)x, rows, cols, ld, esize, em, flag);
    return hbq_check_launch("hbq_flag_nonfinite");
}

}  // extern "C"
