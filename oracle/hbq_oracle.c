/*
 * hbq_oracle.c -- CPU restatement of HBQ's quantize-dequantize and block-quant
 * GEMM semantics.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker: tests/, the smoke()
 * entry point and bench.py's cpu_baseline leg may call it; the product path
 * (hbq_amd/) never links, imports or falls back to it.
 *
 * Every routine restates the arithmetic of the reference step by step, with
 * each tensor operation rounded separately to the tensor dtype T (fp16, bf16
 * or fp32).  PyTorch evaluates fp16/bf16 elementwise ops in fp32 and rounds
 * the result to T; for + - * / of two T values that double rounding equals a
 * single correct rounding (24 >= 2p+2), so each step below is "compute in
 * float, round to T".  No floating-point contraction is allowed anywhere
 * (build with -ffp-contract=off; x86-64 baseline has no FMA anyway).
 *
 * Reference files (SeoLabCornell/HBQ):
 *   src/quantizer.py:148-185  format constants            -> max_norm/min_norm/min_subnorm
 *   src/quantizer.py:187-257  make_fp_quant (elements)     -> fpq_value(..., rnd=0.5004f)
 *   src/quantizer.py:38-63    its torch.compile'd form     -> fpq_value_fused
 *   src/quantizer.py:259-328  fp_quant (scales)            -> fpq_value(..., rnd=0.5f)
 *   src/quantizer.py:481-511  MXFPQuantizer.get_shared_scale -> mx_pot_scale / nv_fp_scale
 *   src/quantizer.py:513-539  MXFPQuantizer.q              -> orc_mxfp_qdq
 *   src/quantizer.py:735-859  HBQQuantizer.quant_scale / q -> orc_hbq_qdq
 *   blockquant_ext_src/gemm.cu:96-303    gemm_core_kernel<bool>         -> orc_gemm_fp16acc / orc_gemm_fp32acc
 *   blockquant_ext_src/gemm.cu:305-553   gemm_core_kernel_grouped<GK>   -> orc_gemm_grouped
 *   blockquant_ext_src/gemm.cu:669-1035  e3m4 psum quant (mxfp8)        -> orc_gemm_mxfp8
 *   blockquant_ext_src/gemm.cu:1137-1396 int8 psum quant (mxint8)       -> orc_gemm_mxint8
 *
 * torch's fp32 accumulation order inside Half/BFloat16 `sum` (used by the
 * HBQ error search, src/quantizer.py:802,814) is restated in cascade_sum()
 * and row_sum(); tests/test_oracle_torch_pins.py pins both against torch.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define DT_F16 0
#define DT_BF16 1
#define DT_F32 2

/* ------------------------------------------------------------------------- */
/* bit-level conversions (IEEE round-to-nearest-even, subnormals kept)        */
/* ------------------------------------------------------------------------- */
static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static inline float h2f(uint16_t h) {
    uint32_t s = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0x1f) return bits_f32(s | 0x7f800000u | (m << 13));
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-08f; /* m * 2^-24, exact */
        return s ? -v : v;
    }
    return bits_f32(s | ((e + 112u) << 23) | (m << 13));
}

static inline uint16_t f2h(float f) {
    uint32_t x = f32_bits(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return sign | 0x7e00u | (uint16_t)((ax >> 13) & 0x3ffu);
    if (ax >= 0x477ff000u) return sign | 0x7c00u;          /* >= 65520 -> inf */
    if (ax >= 0x38800000u) {                                /* normal fp16 */
        uint32_t r = ax + 0xfffu + ((ax >> 13) & 1u);
        r -= 0x38000000u;
        return sign | (uint16_t)(r >> 13);
    }
    float v = bits_f32(ax) * 16777216.0f;                   /* units of 2^-24 */
    return sign | (uint16_t)nearbyintf(v);
}

static inline float bf2f(uint16_t b) { return bits_f32((uint32_t)b << 16); }
static inline uint16_t f2bf(float f) {
    uint32_t x = f32_bits(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

/* round a float to the tensor dtype and return it as float */
static inline float rT(float v, int dt) {
    if (dt == DT_F16) return h2f(f2h(v));
    if (dt == DT_BF16) return bf2f(f2bf(v));
    return v;
}

static inline float ld(const void *p, int64_t i, int dt) {
    if (dt == DT_F32) return ((const float *)p)[i];
    uint16_t b = ((const uint16_t *)p)[i];
    return dt == DT_F16 ? h2f(b) : bf2f(b);
}
static inline void st(void *p, int64_t i, int dt, float v) {
    if (dt == DT_F32) ((float *)p)[i] = v;
    else ((uint16_t *)p)[i] = dt == DT_F16 ? f2h(v) : f2bf(v);
}

/* floor(R_T(log2 v)): torch computes log2 in fp32 and rounds to T
 * (src/quantizer.py:217,291,493-499).  The correctly rounded fp32 log2 is
 * produced via double; tests pin it against torch.log2 for every fp16 and
 * bf16 value. */
static inline float log2_T(float v, int dt) { return rT((float)log2((double)v), dt); }

/* ------------------------------------------------------------------------- */
/* format constants (src/quantizer.py:148-185)                                */
/* ------------------------------------------------------------------------- */
static double max_norm(int ebit, int mbit) {
    if (ebit == 0) return (double)((1 << (mbit - 1)) - 1);
    if (ebit == 4 && mbit == 3) return 448.0;
    int emax = (ebit == 5) ? 15 : (1 << (ebit - 1));
    return ldexp(1.0, emax) * (double)((1 << (mbit + 1)) - 1) / (double)(1 << mbit);
}
static double min_norm(int ebit, int mbit) {
    (void)mbit;
    if (ebit == 0) return 0.0;
    if (ebit == 1) return 1.0;
    return ldexp(1.0, 2 - (1 << (ebit - 1)));
}
static double min_subnorm(int ebit, int mbit) {
    return ldexp(1.0, 2 - (1 << (ebit - 1))) * ldexp(1.0, -mbit);
}

typedef struct {
    int ebit, mbit;
    float emax, emin, min_norm, thr, mmax, mshift;
    int is_e4m3;
} fmt_t;

static void fmt_init(fmt_t *f, int ebit, int mbit) {
    int emax = (ebit == 5) ? 15 : (1 << (ebit - 1));
    int emin = 2 - (1 << (ebit - 1));
    f->ebit = ebit; f->mbit = mbit;
    f->emax = (float)emax; f->emin = (float)emin;
    f->min_norm = (float)min_norm(ebit, mbit);
    f->thr = (float)(min_norm(ebit, mbit) - ldexp(1.0, -(mbit + 1)) * ldexp(1.0, emin));
    f->mmax = (float)((1 << mbit) - 1);
    f->mshift = (float)(1 << mbit);
    f->is_e4m3 = (ebit == 4 && mbit == 3);
}

static inline float sign_of(float x) { return x > 0.f ? 1.f : (x < 0.f ? -1.f : (x != x ? x : 0.f)); }

/*
 * One value through make_fp_quant (rnd = 0.5004f, src/quantizer.py:202-255) or
 * fp_quant (rnd = 0.5f, src/quantizer.py:259-328).  Both share the mask logic;
 * they differ only in the rounding constant.  Returns the value in T.
 */
static float fpq_value(float x, const fmt_t *f, int dt, float rnd, int allow_sub, int use_ceil) {
    float a = fabsf(x);
    int is_zero = (x == 0.f);
    int promote = (a < f->min_norm) && (a >= f->thr);
    int sub = allow_sub && (a < f->thr) && !is_zero;
    int under = !allow_sub && (a < f->thr) && !is_zero;

    float fe = floorf(log2_T(rT(a + (is_zero ? 1.f : 0.f), dt), dt));
    float e = fe < f->emin ? f->emin : (fe > f->emax ? f->emax : fe);   /* clip keeps NaN */
    float p2 = rT(exp2f(e), dt);
    float sg = sign_of(x);
    float mant;
    if (sub) mant = rT(rT(x / p2, dt) * f->mshift, dt);
    else mant = rT(rT(rT(x / p2, dt) - sg, dt) * f->mshift, dt);

    /* the Python scalar is rounded to T before the add (fp16: 0.5004 -> 0.50048828125) */
    float mr = use_ceil ? ceilf(fabsf(mant)) : floorf(rT(fabsf(mant) + rT(rnd, dt), dt));
    int overflow = (mr > f->mmax) && (e != f->emax);
    if (mr > f->mmax) mr = f->mmax;
    if (is_zero || under || overflow || promote) mr = 0.f;
    if (overflow) e = e + 1.f;

    float smant = sg * mr;
    float p2b = rT(exp2f(e), dt);
    float xq;
    if (sub) xq = rT(rT(smant / f->mshift, dt) * p2b, dt);
    else xq = rT(rT(rT(smant / f->mshift, dt) + sg, dt) * p2b, dt);
    if (is_zero || under) xq = 0.f;
    if (f->is_e4m3) xq = xq > 448.f ? 448.f : (xq < -448.f ? -448.f : xq);
    return xq;
}

/*
 * make_fp_quant's callable as GLOBAL_FP_QUANT_CACHE serves it
 * (src/quantizer.py:38-63): torch.compile(fullgraph=True) fuses the whole
 * function (src/quantizer.py:202-255) into one kernel that loads the T value,
 * computes every step in fp32 and rounds to T only at the store.  The comment
 * at src/quantizer.py:224-228 describes exactly this difference from the eager
 * op sequence.  So here, unlike fpq_value:
 *   - floor(log2|x|) is taken in fp32: the exact floor for a 16-bit value (its
 *     fp32 log2 lies at least 2^-12 below the next integer, far above the fp32
 *     spacing there), taken from the binade;
 *   - the mantissa rounding is floor(f32(|m| + f32(0.5004))), with the fp32
 *     constant 0x3F001A37 and no rounding of the sum to T;
 *   - the .to(x.dtype) of that sum is a cast of an fp16-typed value to its own
 *     dtype, which the compiled graph drops.
 * |m| itself is exact in fp32 on both routes.  For fp32 tensors the eager op
 * sequence is already all fp32, so both routes coincide and fp32 uses fpq_value.
 * Pinned by tests/golden/compiled_quant.npz (exhaustive over all 16-bit inputs).
 */
static float fpq_value_fused(float x, const fmt_t *f, int dt) {
    if (dt == DT_F32) return fpq_value(x, f, dt, 0.5004f, 1, 0);
    float a = fabsf(x);
    int is_zero = (x == 0.f);
    int promote = (a < f->min_norm) && (a >= f->thr);
    int sub = (a < f->thr) && !is_zero;
    float fe;
    if (is_zero) fe = 0.f;                       /* log2(|0| + 1) */
    else if (a != a || a == INFINITY) fe = a;    /* log2 of NaN / inf */
    else { int ex; frexpf(a, &ex); fe = (float)(ex - 1); }
    float e = fe < f->emin ? f->emin : (fe > f->emax ? f->emax : fe);   /* clip keeps NaN */
    float p2 = exp2f(e);
    float sg = sign_of(x);
    float mant = sub ? (x / p2) * f->mshift : (x / p2 - sg) * f->mshift;
    volatile float sum = fabsf(mant) + 0.5004f;   /* one fp32 rounding, no contraction */
    float mr = floorf(sum);
    int overflow = (mr > f->mmax) && (e != f->emax);
    if (mr > f->mmax) mr = f->mmax;
    if (is_zero || overflow || promote) mr = 0.f;
    if (overflow) e = e + 1.f;
    float smant = sg * mr;
    float p2b = exp2f(e);
    float xq = sub ? (smant / f->mshift) * p2b : (smant / f->mshift + sg) * p2b;
    if (is_zero) xq = 0.f;
    return rT(xq, dt);
}

static inline float elem_value(float x, const fmt_t *f, int dt, int compiled) {
    return compiled ? fpq_value_fused(x, f, dt) : fpq_value(x, f, dt, 0.5004f, 1, 0);
}

/* MX power-of-two shared scale (src/quantizer.py:489-503) */
static float mx_pot_scale(float amax, int dt, int ebit, int sc_ebit, int use_round) {
    float mn = (dt == DT_F32) ? 1.17549435e-38f : 6.103515625e-05f;
    float v = rT(amax + (amax == 0.f ? mn : 0.f), dt);
    float L = log2_T(v, dt);
    float se = use_round ? nearbyintf(L) : floorf(L);
    se = rT(se - (float)(1 << (ebit - 1)), dt);
    float emax = (float)((1 << (sc_ebit - 1)) - 1), emin = (float)(2 - (1 << (sc_ebit - 1)));
    se = se < emin ? emin : (se > emax ? emax : se);
    return rT(exp2f(se), dt);
}

/* clip to the scale format's range, then fp_quant (src/quantizer.py:505-509, 735-739) */
static float fp_scale_quant(float s, int dt, int sc_ebit, int sc_mbit, int allow_sub, int use_ceil) {
    float lo = (float)(allow_sub ? min_subnorm(sc_ebit, sc_mbit) : min_norm(sc_ebit, sc_mbit));
    float hi = (float)max_norm(sc_ebit, sc_mbit);
    s = s < lo ? lo : (s > hi ? hi : s);
    s = rT(s, dt);
    fmt_t f;
    fmt_init(&f, sc_ebit, sc_mbit);
    return fpq_value(s, &f, dt, 0.5f, allow_sub, use_ceil);
}

/* NVFP-style FP shared scale (src/quantizer.py:504-509) */
static float nv_fp_scale(float amax, int dt, int ebit, int mbit, int sc_ebit, int sc_mbit,
                         int allow_sub, int use_ceil) {
    float s = rT(amax / (float)max_norm(ebit, mbit), dt);
    return fp_scale_quant(s, dt, sc_ebit, sc_mbit, allow_sub, use_ceil);
}

/* torch.max(|x|) over a slice: NaN propagates */
static float absmax(const float *v, int n) {
    float m = 0.f;
    for (int i = 0; i < n; ++i) {
        float a = fabsf(v[i]);
        if (a != a) return a;
        if (a > m) m = a;
    }
    return m;
}

/* ------------------------------------------------------------------------- */
/* torch CPU fp32 accumulation order for Half/BFloat16 sum                    */
/* ------------------------------------------------------------------------- */
/* multi-level cascade: sequential 16-element chunks folded into level 1, the
 * level index growing every 16 chunks (torch's multi_row_sum with level step
 * 16 and four levels).  For n <= 16 it is a plain ascending sum. */
static float cascade_sum(const float *v, int64_t n, int64_t stride) {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    int level_power = 4;
    {   /* max(4, ceil_log2(n) / 4) */
        int cl = 0;
        while (((int64_t)1 << cl) < n) ++cl;
        if (cl / 4 > level_power) level_power = cl / 4;
    }
    int64_t step = (int64_t)1 << level_power, mask = step - 1, i = 0;
    while (i + step <= n) {
        for (int64_t j = 0; j < step; ++j, ++i) acc[0] += v[i * stride];
        for (int lv = 1; lv < 4; ++lv) {
            acc[lv] += acc[lv - 1];
            acc[lv - 1] = 0.f;
            if ((i & (mask << (lv * level_power))) != 0) break;
        }
    }
    for (; i < n; ++i) acc[0] += v[i * stride];
    for (int lv = 1; lv < 4; ++lv) acc[0] += acc[lv];
    return acc[0];
}

/* exported for the tests that pin the order against torch.sum */
float orc_cascade_sum(const float *v, int64_t n, int64_t stride) { return cascade_sum(v, n, stride); }

/* four interleaved cascades combined left to right (torch's row_sum) */
static float row_sum(const float *v, int64_t n) {
    int64_t nilp = n / 4;
    float part[4];
    for (int k = 0; k < 4; ++k) part[k] = cascade_sum(v + k, nilp, 4);
    for (int64_t i = nilp * 4; i < n; ++i) part[0] += v[i];
    float s = part[0];
    for (int k = 1; k < 4; ++k) s += part[k];
    return s;
}

float orc_row_sum(const float *v, int64_t n) { return row_sum(v, n); }

/* ------------------------------------------------------------------------- */
/* exported scalar tables                                                     */
/* ------------------------------------------------------------------------- */
int orc_elem_quant(const void *x, void *y, int64_t n, int dt, int ebit, int mbit, int use_ceil, int compiled) {
    fmt_t f;
    fmt_init(&f, ebit, mbit);
    if (compiled && use_ceil) return -1;   /* the cache only serves use_ceil=False */
    for (int64_t i = 0; i < n; ++i)
        st(y, i, dt, compiled ? fpq_value_fused(ld(x, i, dt), &f, dt)
                              : fpq_value(ld(x, i, dt), &f, dt, 0.5004f, 1, use_ceil));
    return 0;
}

int orc_fp_quant(const void *x, void *y, int64_t n, int dt, int ebit, int mbit, int allow_sub, int use_ceil) {
    fmt_t f;
    fmt_init(&f, ebit, mbit);
    for (int64_t i = 0; i < n; ++i) st(y, i, dt, fpq_value(ld(x, i, dt), &f, dt, 0.5f, allow_sub, use_ceil));
    return 0;
}

int orc_floor_log2(const void *x, float *y, int64_t n, int dt) {
    for (int64_t i = 0; i < n; ++i) y[i] = floorf(log2_T(fabsf(ld(x, i, dt)), dt));
    return 0;
}

int orc_mx_scale(const void *amax, void *y, int64_t n, int dt, int ebit, int mbit, int sc_ebit, int sc_mbit,
                 int allow_sub, int use_round, int use_ceil) {
    for (int64_t i = 0; i < n; ++i) {
        float a = ld(amax, i, dt);
        float s = sc_mbit == 0 ? mx_pot_scale(a, dt, ebit, sc_ebit, use_round)
                               : nv_fp_scale(a, dt, ebit, mbit, sc_ebit, sc_mbit, allow_sub, use_ceil);
        st(y, i, dt, s);
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* MXFPQuantizer.q  (src/quantizer.py:513-539), blocks along the last dim,    */
/* zero padded to a multiple of the block (src/quantizer.py:67-146)           */
/* ------------------------------------------------------------------------- */
int orc_mxfp_qdq(const void *x, void *y, void *scale_out, int64_t rows, int64_t cols, int dt,
                 int block, int ebit, int mbit, int sc_ebit, int sc_mbit, int allow_sub,
                 int use_round, int use_ceil, int per_tensor, double tensor_scale, int compiled) {
    if (block <= 0 || block > 4096) return -1;
    int64_t nblk = (cols + block - 1) / block;
    fmt_t f;
    fmt_init(&f, ebit, mbit);
    /* python float scalars are rounded to T before the op (src/quantizer.py:524,535) */
    float ts = rT((float)tensor_scale, dt);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        float v[4096];
        for (int64_t b = 0; b < nblk; ++b) {
            for (int i = 0; i < block; ++i) {
                int64_t c = b * block + i;
                float xv = c < cols ? ld(x, r * cols + c, dt) : 0.f;
                v[i] = per_tensor ? rT(xv / ts, dt) : xv;
            }
            float amax = absmax(v, block);
            float s = sc_mbit == 0 ? mx_pot_scale(amax, dt, ebit, sc_ebit, use_round)
                                   : nv_fp_scale(amax, dt, ebit, mbit, sc_ebit, sc_mbit, allow_sub, use_ceil);
            if (scale_out) st(scale_out, r * nblk + b, dt, s);
            for (int i = 0; i < block; ++i) {
                int64_t c = b * block + i;
                if (c >= cols) break;
                float yv = rT(v[i] / s, dt);
                float q = elem_value(yv, &f, dt, compiled);
                float o = rT(q * s, dt);
                if (per_tensor) o = rT(o * ts, dt);
                st(y, r * cols + c, dt, o);
            }
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* HBQQuantizer  (src/quantizer.py:704-859)                                   */
/* ------------------------------------------------------------------------- */
enum { SCH_POT = 0, SCH_INT, SCH_SIG1, SCH_FPM1, SCH_FP1, SCH_FPM10, SCH_FPM100, SCH_MIX };

/* L2 candidate table l2[j*S + s] in T (src/quantizer.py:745-770); returns S */
int orc_hbq_l2_table(int scheme, int l2_sc_bit, int dt, float *tab) {
    int J = 1 << l2_sc_bit;
    float d1 = (float)(1 << l2_sc_bit), d2 = (float)(1 << (l2_sc_bit + 1)), d3 = (float)(1 << (l2_sc_bit + 2));
    for (int r = 0; r < J; ++r) {
        float rr = (float)r;
        float pot = rT(exp2f(rr), dt);
        float in = rT(rr + 1.f, dt);
        float sig = rT(1.f + rT(rr / 2.f, dt), dt);
        float fp = rT(1.f + rT(rr / d1, dt), dt);
        float fp1 = rT(1.f + rT(rT(rr + 1.f, dt) / d1, dt), dt);
        float fp10 = rT(1.f + rT(rr / d2, dt), dt);
        float fp100 = rT(1.f + rT(rr / d3, dt), dt);
        switch (scheme) {
            case SCH_POT: tab[r] = pot; break;
            case SCH_INT: tab[r] = in; break;
            case SCH_SIG1: tab[r] = sig; break;
            case SCH_FPM1: tab[r] = fp; break;
            case SCH_FP1: tab[r] = fp1; break;
            case SCH_FPM10: tab[r] = fp10; break;
            case SCH_FPM100: tab[r] = fp100; break;
            case SCH_MIX: tab[r * 2 + 0] = fp; tab[r * 2 + 1] = fp10; break;
            default: return -1;
        }
    }
    return scheme == SCH_MIX ? 2 : 1;
}

/* argmin with torch semantics: first minimum; a NaN wins and the first NaN is kept */
static inline int better(float v, float best) { return (v != v) ? (best == best) : (v < best); }

#define HBQ_MAXB 1024
#define HBQ_MAXJ 16
#define HBQ_MAXS 2

int orc_hbq_qdq(const void *x, void *y, void *l1_out, uint8_t *l2idx_out, uint8_t *scheme_out,
                void *l2val_out, int64_t rows, int64_t cols, int dt, int block, int ebit, int mbit,
                int sc_ebit, int sc_mbit, int l2b, int l2_sc_bit, int scheme, int allow_sub, int use_ceil,
                int compiled) {
    if (block <= 0 || block > HBQ_MAXB || l2b <= 0 || block % l2b) return -1;
    if (l2_sc_bit < 0 || (1 << l2_sc_bit) > HBQ_MAXJ) return -1;
    float tab[HBQ_MAXJ * HBQ_MAXS];
    int S = orc_hbq_l2_table(scheme, l2_sc_bit, dt, tab);
    if (S < 0) return -1;
    int J = 1 << l2_sc_bit;
    int nsub = block / l2b;
    int64_t nblk = (cols + block - 1) / block;
    fmt_t f;
    fmt_init(&f, ebit, mbit);
    /* em[s] = R_T(ele_max * max_j l2[j, s])  (src/quantizer.py:775-777) */
    float em[HBQ_MAXS];
    float elemax = rT((float)max_norm(ebit, mbit), dt);
    for (int s = 0; s < S; ++s) {
        float m = tab[s];
        for (int j = 1; j < J; ++j) if (tab[j * S + s] > m) m = tab[j * S + s];
        em[s] = rT(elemax * m, dt);
    }
    int rc = 0;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        float xv[HBQ_MAXB];
        float *d = malloc(sizeof(float) * HBQ_MAXB * HBQ_MAXJ * HBQ_MAXS);
        float *sq = malloc(sizeof(float) * HBQ_MAXB * HBQ_MAXJ * HBQ_MAXS);
        float sel[HBQ_MAXB];
        int jbest[HBQ_MAXB / 1][HBQ_MAXS];
        for (int64_t b = 0; b < nblk; ++b) {
            for (int i = 0; i < block; ++i) {
                int64_t c = b * block + i;
                xv[i] = c < cols ? ld(x, r * cols + c, dt) : 0.f;
            }
            float amax = absmax(xv, block);
            float l1[HBQ_MAXS];
            for (int s = 0; s < S; ++s)
                l1[s] = fp_scale_quant(rT(amax / em[s], dt), dt, sc_ebit, sc_mbit, allow_sub, use_ceil);
            /* candidates: d[(i*J + j)*S + s] */
            for (int i = 0; i < block; ++i)
                for (int s = 0; s < S; ++s) {
                    float t = rT(xv[i] / l1[s], dt);
                    for (int j = 0; j < J; ++j) {
                        float l2 = tab[j * S + s];
                        float u = rT(t / l2, dt);
                        float q = elem_value(u, &f, dt, compiled);
                        float dq = rT(rT(q * l2, dt) * l1[s], dt);
                        float e = fabsf(rT(xv[i] - dq, dt));
                        d[(i * J + j) * S + s] = dq;
                        sq[(i * J + j) * S + s] = rT(e * e, dt);
                    }
                }
            /* sub-block search (src/quantizer.py:799-803) */
            for (int u = 0; u < nsub; ++u)
                for (int s = 0; s < S; ++s) {
                    int bj = 0;
                    float best = 0.f;
                    for (int j = 0; j < J; ++j) {
                        const float *base = sq + ((int64_t)(u * l2b) * J + j) * S + s;
                        float e = rT(cascade_sum(base, l2b, (int64_t)J * S), dt);
                        if (j == 0 || better(e, best)) { best = e; bj = j; }
                    }
                    jbest[u][s] = bj;
                }
            /* scheme search (src/quantizer.py:811-816) */
            int bs = 0;
            float bse = 0.f;
            for (int s = 0; s < S; ++s) {
                for (int i = 0; i < block; ++i) sel[i] = sq[((int64_t)i * J + jbest[i / l2b][s]) * S + s];
                float e = rT(row_sum(sel, block), dt);
                if (s == 0 || better(e, bse)) { bse = e; bs = s; }
            }
            for (int i = 0; i < block; ++i) {
                int64_t c = b * block + i;
                if (c < cols) st(y, r * cols + c, dt, d[((int64_t)i * J + jbest[i / l2b][bs]) * S + bs]);
            }
            if (l1_out) st(l1_out, r * nblk + b, dt, l1[bs]);
            if (scheme_out) scheme_out[r * nblk + b] = (uint8_t)bs;
            for (int u = 0; u < nsub; ++u) {
                int64_t o = (r * nblk + b) * nsub + u;
                if (l2idx_out) l2idx_out[o] = (uint8_t)jbest[u][bs];
                if (l2val_out) st(l2val_out, o, dt, tab[jbest[u][bs] * S + bs]);
            }
        }
        free(d);
        free(sq);
    }
    return rc;
}

/* ------------------------------------------------------------------------- */
/* GEMM semantics of blockquant_ext (gemm.cu).  A [M,K], B [K,N] fp16 row-   */
/* major, C [M,N] fp16.  fmaf() is the correctly rounded fused fp32 FMA.      */
/* ------------------------------------------------------------------------- */
static inline float hadd(float a, float b) { return h2f(f2h(a + b)); }  /* fp16 add: exact sum rounded once */

/* fp16 fused multiply-add with one rounding: a*b + c exactly, then RNE.
 * fp16 values are integer multiples of 2^-24, so a*b + c is an integer
 * multiple of 2^-48 below 2^81: __int128 holds it exactly. */
static float hfma(uint16_t a, uint16_t b, uint16_t c) {
    float fa = h2f(a), fb = h2f(b), fc = h2f(c);
    if (!isfinite(fa) || !isfinite(fb) || !isfinite(fc)) return h2f(f2h(fa * fb + fc));
    __int128 ia = (__int128)llrint((double)fa * 16777216.0);
    __int128 ib = (__int128)llrint((double)fb * 16777216.0);
    __int128 ic = (__int128)llrint((double)fc * 16777216.0);
    __int128 v = ia * ib + (ic << 24);            /* units of 2^-48 */
    if (v == 0) {
        /* exact zero: sign per IEEE (+0 unless both addends are -0) */
        int prod_neg = (signbit(fa) != 0) != (signbit(fb) != 0);
        int c_neg = signbit(fc) != 0;
        return (prod_neg && c_neg) ? -0.f : 0.f;
    }
    int neg = v < 0;
    unsigned __int128 m = neg ? (unsigned __int128)(-v) : (unsigned __int128)v;
    /* target quantum: max(2^-24, ulp of the fp16 binade) expressed in 2^-48 units */
    int msb = 127;
    while (!((m >> msb) & 1)) --msb;
    int e = msb - 48;                 /* value in [2^e, 2^(e+1)) */
    int q = (e < -14 ? -24 : e - 10) + 48;   /* log2 of quantum in 2^-48 units */
    unsigned __int128 unit = (unsigned __int128)1 << q;
    unsigned __int128 k = m >> q, rem = m & (unit - 1), half = unit >> 1;
    if (rem > half || (rem == half && (k & 1))) ++k;
    double val = ldexp((double)k, q - 48);
    if (val >= 65520.0) val = INFINITY;
    return neg ? -(float)val : (float)val;
}

/* One fp32 fmaf chain per output over ascending k.  The loops run k outside n so B is
 * read along its rows; each output's chain keeps its own order (loop interchange only). */
int orc_gemm_fp32acc(const uint16_t *A, const uint16_t *B, uint16_t *C, int M, int N, int K) {
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; ++m) {
        float *acc = calloc((size_t)N, sizeof(float));
        for (int k = 0; k < K; ++k) {
            const float a = h2f(A[(int64_t)m * K + k]);
            const uint16_t *b = B + (int64_t)k * N;
            for (int n = 0; n < N; ++n) acc[n] = fmaf(a, h2f(b[n]), acc[n]);
        }
        for (int n = 0; n < N; ++n) C[(int64_t)m * N + n] = f2h(acc[n]);
        free(acc);
    }
    return 0;
}

int orc_gemm_fp16acc(const uint16_t *A, const uint16_t *B, uint16_t *C, int M, int N, int K) {
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            uint16_t acc = 0;
            for (int k = 0; k < K; ++k) acc = f2h(hfma(A[(int64_t)m * K + k], B[(int64_t)k * N + n], acc));
            C[(int64_t)m * N + n] = acc;
        }
    return 0;
}

/* fp32 partial of one K group, sequential fmaf over ascending k */
static inline float group_partial(const uint16_t *A, const uint16_t *B, int N, int K, int m, int n, int k0, int k1) {
    float p = 0.f;
    for (int k = k0; k < k1; ++k) p = fmaf(h2f(A[(int64_t)m * K + k]), h2f(B[(int64_t)k * N + n]), p);
    return p;
}

/* int8 psum quantize-dequantize of one (row, GN columns) slice, in place (gemm.cu:1145-1251) */
static void psum_int8(float *p, int gn) {
    float mx = 0.f;
    for (int i = 0; i < gn; ++i) { float a = fabsf(p[i]); if (a > mx) mx = a; }
    float scale = mx <= 0.f ? 1.f : ldexpf(1.f, ilogbf(mx) - 6);
    if (mx > 0.f && isinf(mx)) scale = INFINITY;
    float inv = 1.f / scale;
    for (int i = 0; i < gn; ++i) {
        float v = p[i] * inv;
        if (!isfinite(v)) {
            if (isnan(v)) { p[i] = NAN; continue; }
            v = copysignf(127.f, v);
        }
        float q = nearbyintf(v);
        if (q > 127.f) q = 127.f;
        if (q < -127.f) q = -127.f;
        p[i] = q * scale;
    }
}

/* E3M4 quantize-dequantize with a power-of-two scale (gemm.cu:677-745).
 * The exponent is the exact floor(log2 y) (the reference's fast-math log2f
 * may differ a few ulps below powers of two; parity unpinned there). */
static float e3m4_qdq(float x, float scale) {
    float sgn = copysignf(1.f, x);
    float a = fabsf(x);
    if (a == 0.f) return copysignf(0.f, x);
    float y = a / scale;
    if (!isfinite(y)) {
        if (isnan(y)) return copysignf(NAN, x);
        return sgn * 15.5f * scale;
    }
    if (y < 0.5f * 0.015625f) return 0.f;
    if (y >= 0.25f) {
        int e = ilogbf(y);
        if (e < -2) e = -2;
        if (e > 3) e = 3;
        float p2 = ldexpf(1.f, e);
        float frac = y / p2 - 1.f;
        float mant = nearbyintf(frac * 16.f);
        if (mant >= 16.f) {
            mant = 0.f;
            ++e;
            if (e > 3) { e = 3; mant = 15.f; }
            p2 = ldexpf(1.f, e);
        }
        float yq = (1.f + mant * (1.f / 16.f)) * p2;
        if (yq > 15.5f) yq = 15.5f;
        return sgn * yq * scale;
    }
    float mant = nearbyintf(y * 64.f);
    if (mant <= 0.f) return 0.f;
    if (mant >= 16.f) return sgn * 0.25f * scale;
    float yq = (mant * (1.f / 16.f)) * 0.25f;
    return sgn * yq * scale;
}

static void psum_e3m4(float *p, int gn) {
    float mx = 0.f;
    for (int i = 0; i < gn; ++i) { float a = fabsf(p[i]); if (a > mx) mx = a; }
    float scale = mx <= 0.f ? 1.f : (isinf(mx) ? INFINITY : ldexpf(1.f, ilogbf(mx) - 3));
    for (int i = 0; i < gn; ++i) p[i] = e3m4_qdq(p[i], scale);
}

/*
 * Cross-group epilogues applied to given fp32 group partials P[g][m][n]:
 * mode 0 = grouped fp16 accumulation (gemm.cu:354-377), 1 = int8 psum quant,
 * 2 = E3M4 psum quant (quant modes use column groups of gn).
 */
int orc_epilogue(const float *P, uint16_t *C, int G, int M, int N, int mode, int gn) {
    if (mode != 0 && (gn <= 0 || N % gn)) return -1;
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; ++m) {
        float *row = malloc(sizeof(float) * (size_t)N);
        float *H = malloc(sizeof(float) * (size_t)N);
        for (int n = 0; n < N; ++n) H[n] = 0.f;
        for (int g = 0; g < G; ++g) {
            memcpy(row, P + ((int64_t)g * M + m) * N, sizeof(float) * (size_t)N);
            if (mode == 1) for (int c = 0; c < N; c += gn) psum_int8(row + c, gn);
            if (mode == 2) for (int c = 0; c < N; c += gn) psum_e3m4(row + c, gn);
            for (int n = 0; n < N; ++n) H[n] = hadd(H[n], h2f(f2h(row[n])));
        }
        for (int n = 0; n < N; ++n) C[(int64_t)m * N + n] = f2h(H[n]);
        free(row);
        free(H);
    }
    return 0;
}

/* group partials P[g][m][n] with groups of gk along K; the tail group ends at K.  Each
 * partial is group_partial()'s sequential fmaf chain; the loops run k outside n so B is
 * read along its rows (loop interchange only: every chain keeps its ascending order). */
int orc_group_partials(const uint16_t *A, const uint16_t *B, float *P, int M, int N, int K, int gk) {
    int G = (K + gk - 1) / gk;
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; ++m)
        for (int g = 0; g < G; ++g) {
            int k0 = g * gk, k1 = k0 + gk < K ? k0 + gk : K;
            float *p = P + ((int64_t)g * M + m) * N;
            for (int n = 0; n < N; ++n) p[n] = 0.f;
            for (int k = k0; k < k1; ++k) {
                const float a = h2f(A[(int64_t)m * K + k]);
                const uint16_t *b = B + (int64_t)k * N;
                for (int n = 0; n < N; ++n) p[n] = fmaf(a, h2f(b[n]), p[n]);
            }
        }
    return 0;
}

/* the partial of one (m, n): kept as the plain statement of the chain above; the tests
 * compare both */
float orc_group_partial_one(const uint16_t *A, const uint16_t *B, int N, int K, int m, int n, int k0, int k1) {
    return group_partial(A, B, N, K, m, n, k0, k1);
}

static int gemm_grouped_mode(const uint16_t *A, const uint16_t *B, uint16_t *C, int M, int N, int K, int gk,
                             int mode, int gn) {
    int G = (K + gk - 1) / gk;
    float *P = malloc(sizeof(float) * (size_t)G * (size_t)M * (size_t)N);
    if (!P) return -2;
    orc_group_partials(A, B, P, M, N, K, gk);
    int rc = orc_epilogue(P, C, G, M, N, mode, gn);
    free(P);
    return rc;
}

int orc_gemm_grouped(const uint16_t *A, const uint16_t *B, uint16_t *C, int M, int N, int K, int gk) {
    return gemm_grouped_mode(A, B, C, M, N, K, gk, 0, 0);
}
int orc_gemm_mxint8(const uint16_t *A, const uint16_t *B, uint16_t *C, int M, int N, int K, int gk, int gn) {
    if (K % gk) return -1;
    return gemm_grouped_mode(A, B, C, M, N, K, gk, 1, gn);
}
int orc_gemm_mxfp8(const uint16_t *A, const uint16_t *B, uint16_t *C, int M, int N, int K, int gk, int gn) {
    if (K % gk) return -1;
    return gemm_grouped_mode(A, B, C, M, N, K, gk, 2, gn);
}
