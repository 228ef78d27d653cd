// Table-driven HBQ quantize-dequantize (fp16 / bf16 inputs, the configurations
// of the HBQ-A/E formats).
//
// After the L1 division t = R_T(|x| / l1) the rest of the candidate chain of
// HBQQuantizer.q (src/quantizer.py:781-791) depends on t alone: for every L2
// candidate j the element level of R_T(t / l2_j) is a fixed function of the
// 16-bit value t.  So
//   * a level table indexed by the bits of t (the binades where the level is
//     not constant) holds the levels of all J <= 4 candidates in one 32-bit
//     word; it is built once per device and configuration on the GPU with the
//     same device element quantizer as the generic kernel, and copied to LDS
//     by each (persistent) workgroup;
//   * per block, the dequantized magnitudes R_T(R_T(level * l2_j) * l1) of
//     every (scheme, candidate, level) are tabulated in LDS by the block's lanes.
// Per element and candidate what remains is the exact error arithmetic of the
// reference: e = R_T(|x| - d), sq = R_T(e^2), and the fp32 sub-block sums in
// torch's order (src/quantizer.py:802).  Signs never change an error, so the
// candidate search runs on magnitudes; the sign of the output follows the
// reference's zero rules (src/quantizer.py:241-245).
#include <hip/hip_runtime.h>
#include <math.h>
#include <mutex>
#include <type_traits>
#include <stdint.h>
#include <string.h>

#include "hbq_capi_internal.h"
#include "hbq_fast.h"
#include "model_math.h"
#include "quant_common.h"

namespace hbq {

constexpr int kLutSlots = 16;
constexpr int kLutMaxBinades = 12;
constexpr int kLutMaxEntries = 2 * (kLutMaxBinades * 1024 + 2);
static_assert(kLutMaxEntries % 4 == 0, "the table copy reads whole 16-byte pieces of a slot row");
constexpr int kFastJ = 4;

// level tables: per slot, S schemes of (n + 2) words: [0] below the table range
// (all levels 0), [1 .. n] the binades [2^lo, 2^hi), [n + 1] at or above 2^hi
// (saturated).  Byte j of a word is candidate j's level times the element size
// of the magnitude table, i.e. its byte offset in a table row.
static __device__ __attribute__((aligned(16))) uint32_t g_lut[kLutSlots][kLutMaxEntries];
// per slot: z[s][j] = smallest t > 0 with R_T(t / l2[j][s]) != 0
static __device__ float g_lut_z[kLutSlots][2 * kFastJ];
// per slot: R_T(level value * l2[j][s]) for every level (block independent)
static __device__ float g_lut_qs[kLutSlots][2][kFastJ][32];
static __device__ int g_lut_status[kLutSlots];
// 1 when v_rcp_f32 returns the correctly rounded 1 / l1 for every E5M3 L1 scale the
// table kernel can produce (2^e (1 + m / 8), e in [-14, 15]); set by the table build
static __device__ int g_rcp_exact;

struct FastParams {
    int S, J, L;               // schemes, candidates, levels (2^(m+2))
    int n;                     // table words per scheme, sentinels excluded
    uint32_t lo_bits;          // T bit pattern of 2^lo
    float l2[kFastJ][2];       // L2 factors
    float em[2];
    float rem[2];              // R32(1 / em): R_T(amax * rem) equals R_T(amax / em) wherever the clamp below keeps it
    int use_ceil;
    int fused;                 // the table's element rounding: compiled lpfp_quant (1) or eager (0)
};

// fp16 tables hold halves (the candidate errors are computed in packed fp16),
// bf16 tables hold floats
template <class T>
using DTabT = typename std::conditional<T::dt == kF16, _Float16, float>::type;
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

// bit pattern of a value already representable in T
template <class T>
__device__ __forceinline__ uint32_t bits_of(float v) {
    if (T::dt == kBF16) return f2bits(v) >> 16;
    return (uint32_t)T::store(v);
}

// ordering key of a value already representable in T: its bit pattern shifted
// left by 16 for bf16 (the float's own bits, low half zero), as is for fp16
template <class T>
__device__ __forceinline__ uint32_t key_of(float v) {
    if (T::dt == kBF16) return f2bits(v);
    return (uint32_t)T::store(v);
}

template <class T>
__device__ __forceinline__ float from_bits(uint32_t b) {
    return T::load((typename T::storage)b);
}

// magnitude code of the element quantizer = its level (exponent field and mantissa)
template <class T, int M>
__device__ __forceinline__ uint32_t level_of(float u, bool fused) {
    uint32_t c;
    elem_quant<T, M>(u, c, fused);
    return c & ((1u << (M + 2)) - 1u);
}

template <int M>
__device__ __forceinline__ float level_value(int c) {
    const int ef = c >> M, mf = c & ((1 << M) - 1);
    return ef == 0 ? (float)mf * (1.0f / (float)(1 << M))
                   : (1.0f + (float)mf * (1.0f / (float)(1 << M))) * pow2f(ef - 1);
}

template <class T, int M>
__global__ void build_lut_kernel(int slot, FastParams p) {
    constexpr uint32_t esize = sizeof(DTabT<T>);
    const int per = p.n + 2;
    const int total = p.S * per;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
        const int s = i / per, k = i % per;
        uint32_t w = 0;
        if (k == per - 1) {
            for (int j = 0; j < p.J; ++j) w |= (((1u << (M + 2)) - 1u) * esize) << (8 * j);
        } else if (k > 0) {
            const float t = from_bits<T>(p.lo_bits + (uint32_t)(k - 1));
            for (int j = 0; j < p.J; ++j)
                w |= (level_of<T, M>(T::round(t / p.l2[j][s]), p.fused) * esize) << (8 * j);
        }
        g_lut[slot][i] = w;
    }
    const int g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g < 2 * kFastJ * 32) {
        const int s = g / (kFastJ * 32), j = (g / 32) % kFastJ, c = g % 32;
        const float l2 = (s < p.S && j < p.J) ? p.l2[j][s] : 1.0f;
        g_lut_qs[slot][s][j][c] = c < (1 << (M + 2)) ? T::round(level_value<M>(c) * l2) : 0.0f;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        int status = 0;
        // the constant ends of the table: the largest value below 2^lo has level 0,
        // 2^hi is already saturated, for every candidate
        const float below = from_bits<T>(p.lo_bits - 1u);
        const float top = from_bits<T>(p.lo_bits + (uint32_t)p.n);
        for (int s = 0; s < p.S; ++s)
            for (int j = 0; j < p.J; ++j) {
                if (level_of<T, M>(T::round(below / p.l2[j][s]), p.fused) != 0) status = 1;
                if (level_of<T, M>(T::round(top / p.l2[j][s]), p.fused) != (1u << (M + 2)) - 1u) status = 2;
                float z = -1.f;
                for (uint32_t b = 1; b < 4096 && z < 0.f; ++b) {
                    const float t = from_bits<T>(b);
                    if (T::round(t / p.l2[j][s]) != 0.f) z = t;
                }
                if (z < 0.f) status = 3;
                g_lut_z[slot][s * kFastJ + j] = z;
            }
        g_lut_status[slot] = status;
        int exact = 1;
        for (int e = -14; e <= 15; ++e)
            for (int m = 0; m < 8; ++m) {
                float v = ldexpf(1.0f + 0.125f * (float)m, e);
                asm volatile("" : "+v"(v));   // the hardware's reciprocal, not a folded constant
                if (__builtin_amdgcn_rcpf(v) != 1.0f / v) exact = 0;
            }
        g_rcp_exact = exact;
    }
}

// Workgroup size: the fp16 level table (1024 words a binade) takes 37 KB of LDS,
// which 256-thread workgroups would replicate down to 3 waves a SIMD; 512 threads
// share one copy between 8 waves.  The two tables of the fp16 two-scheme (Mix) E2M1
// kernel take 57 KB: 1024 threads (121 KB of LDS with the magnitude rows, at most 128
// VGPRs) run 4 waves a SIMD where 512 would run 2.  The bf16 table is 8 times smaller.
template <class T, int M, int S>
constexpr int fast_threads() { return T::dt == kF16 ? (S == 2 && M == 1 ? 1024 : 512) : 256; }

// The bf16 two-scheme memory-input kernels run 4 waves a SIMD (128 VGPRs) without the
// input prefetch, whose 8 registers would take them to 3: 12-13% faster than 3 waves
// with it.  The others take what their registers give (a minimum of 1 places no bound).
template <class T, int S>
constexpr bool fast_prefetch() { return !(S == 2 && T::dt == kBF16); }
template <class T, int S, int SRC>
constexpr int fast_min_waves() { return SRC == kSrcX && !fast_prefetch<T, S>() ? 4 : 1; }

// Per-block magnitude rows.  The negated magnitudes fill the second half of each
// row: a level-word byte (level times the entry size) plus L * sizeof(DT) addresses
// -d, so one LDS read of the selected candidate returns the signed output.  Rows are
// padded to start 8 banks apart for the four blocks of a half-wave.
template <class T, int M>
constexpr int fast_row() {
    return 2 * (1 << (M + 2)) + 32 / (int)sizeof(DTabT<T>);
}

// The in-place quantizer of causal attention weights (memory input, causal_t > 0) is
// its own instantiation, so that the plain memory-input kernel can prefetch.
constexpr int kSrcXCausal = 3;

// Block 128 (8 lanes x 16 elements).  Per-wave magnitude tables, laid out
// [scheme][candidate][block-in-wave][row of fast_row() entries].
template <class T, int M, int L2B, int S, int SRC = kSrcX>
__global__ __launch_bounds__((fast_threads<T, M, S>())) __attribute__((amdgpu_waves_per_eu(fast_min_waves<T, S, SRC>())))
void hbq_fast_kernel(const typename T::storage* __restrict__ x,
                                                            typename T::storage* __restrict__ y,
                                                            typename T::storage* __restrict__ l1_out,
                                                            uint8_t* __restrict__ l2i_out,
                                                            uint8_t* __restrict__ sch_out,
                                                            uint8_t* __restrict__ codes, int64_t nb, int64_t causal_t,
                                                            int slot, FastParams p, FastSrc src, int64_t cols) {
    using DT = DTabT<T>;
    constexpr int lpb = 8;
    constexpr int bpw = 64 / lpb;
    constexpr int block = kV * lpb;
    constexpr int L = 1 << (M + 2);
    constexpr int ROW = fast_row<T, M>();              // padded row (entries)
    constexpr int NSUBL = L2B <= kV ? kV / L2B : 1;
    constexpr int LPS = L2B <= kV ? 1 : L2B / kV;
    constexpr int SUBN = L2B <= kV ? L2B : kV;
    constexpr int NTH = fast_threads<T, M, S>();
    constexpr int blocks_per_wg = NTH / lpb;
    extern __shared__ __attribute__((aligned(16))) uint32_t smem[];
    const int per = p.n + 2;
    uint32_t* lut = smem;
    const int li = (int)(threadIdx.x & (lpb - 1));
    const int lane = (int)(threadIdx.x & 63);
    const int lane_base = lane - li;
    const int bw = lane / lpb;
    typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

    // The level table goes to LDS in 16-byte pieces, every global load issued before the
    // first LDS store (a loop with a run-time count waits for each load in turn); the
    // first tile's input loads follow them, so one memory latency covers both.  The
    // slot rows are 16-byte aligned; the up to 3 words copied past the table land in
    // the magnitude rows, which every tile writes before reading.
    constexpr int kCopyWords = S * (kLutMaxBinades * (T::dt == kF16 ? 1024 : 128) + 2);
    constexpr int kCopy = ((kCopyWords + 3) / 4 + NTH - 1) / NTH;
    const int nw4 = (S * per + 3) / 4;
    u32x4_t cp[kCopy];
    {
        const u32x4_t* src4 = reinterpret_cast<const u32x4_t*>(g_lut[slot]);
#pragma unroll
        for (int c = 0; c < kCopy; ++c) {
            const int i = (int)threadIdx.x + c * NTH;
            cp[c] = src4[i < nw4 ? i : nw4 - 1];
        }
    }

    float z[S][kFastJ];
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
        for (int j = 0; j < kFastJ; ++j) z[s][j] = g_lut_z[slot][s * kFastJ + j];
    // this lane builds levels c = li and li + 8 (L = 16) of every (scheme, candidate) row
    // from R_T(level * l2_j).  The two-scheme kernels keep them in LDS after the level
    // table as [li][s][j][k] (a lane's values contiguous) and read them back for each
    // tile, since in registers they would hold 8 * CPL VGPRs for the whole kernel; the
    // one-scheme kernels, whose occupancy does not depend on them, keep them in
    // registers (1-2% faster)
    constexpr int CPL = (L + lpb - 1) / lpb;
    constexpr int QSL = S * kFastJ * CPL;   // floats of one lane
    constexpr bool kQsLds = S == 2;
    float* const qsl = reinterpret_cast<float*>(smem + (S * per + 3) / 4 * 4);
    float qsv = 0.f;
    float qreg[S][kFastJ][CPL];
    if constexpr (kQsLds) {
        qsv = g_lut_qs[slot][(threadIdx.x / (kFastJ * CPL)) % S][(threadIdx.x / CPL) % kFastJ]
                      [((threadIdx.x / QSL) % lpb + (threadIdx.x % CPL) * lpb) & 31];
    } else {
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int j = 0; j < kFastJ; ++j)
#pragma unroll
                for (int k = 0; k < CPL; ++k) qreg[s][j][k] = g_lut_qs[slot][s][j][(li + k * lpb) & 31];
    }

    // this lane's row (s, j) starts at dwave + ((s*J + j)*bpw + bw) * ROW; table words hold byte offsets into it
    DT* dwave = reinterpret_cast<DT*>(kQsLds ? qsl + lpb * QSL : reinterpret_cast<float*>(smem + S * per)) +
                (threadIdx.x >> 6) * (S * kFastJ * bpw * ROW);
    const char* drow0 = reinterpret_cast<const char*>(dwave + bw * ROW);
    const int64_t ntiles = (nb + blocks_per_wg - 1) / blocks_per_wg;
    const float tiny = T::dt == kF16 ? 6.103515625e-05f : 1.17549435e-38f;
    const bool rcp_exact = __builtin_amdgcn_readfirstlane(g_rcp_exact) != 0;

    // causal_t > 0 (kSrcXCausal only): nb blocks of [mats, t, t] attention weights whose
    // blocks above the diagonal are zero and stay as they are (y == x): each wave takes one
    // column block of 8 consecutive rows among the blocks on or below the diagonal.  Rows
    // 128k .. 128k+127 of a matrix (band k, 16 groups of 8 rows) hold k + 1 such blocks.
    if constexpr (SRC != kSrcXCausal) causal_t = 0;
    constexpr bool kMem = SRC == kSrcX || SRC == kSrcXCausal;
    const int64_t nbt = causal_t / block;
    const int64_t per_mat = 8 * nbt * (nbt + 1);
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int64_t nwork = causal_t ? nb / (causal_t * nbt) * per_mat : ntiles;
    const int64_t first = causal_t ? (int64_t)blockIdx.x * (NTH / 64) + wave : (int64_t)blockIdx.x;
    const int64_t stride = causal_t ? (int64_t)gridDim.x * (NTH / 64) : (int64_t)gridDim.x;

    // memory input in row order: the next tile's 16 elements per lane are loaded while this
    // tile is worked on.  No lane branches around the loads (a lane past the end of the
    // last tile reads its current block again and the data is replaced by zeros), and no
    // other path writes their registers, so the compiler waits for them only where the next
    // tile reads them; after the wave's last tile none are issued (a wave-uniform branch).
    constexpr bool kPrefetch = SRC == kSrcX && fast_prefetch<T, S>();
    u32x4_t pf0 = {0u, 0u, 0u, 0u}, pf1 = {0u, 0u, 0u, 0u};
    auto prefetch_load = [&](int64_t t, int64_t g_cur) __attribute__((always_inline)) {
        const int64_t g = t * blocks_per_wg + (threadIdx.x / lpb);
        const u32x4_t* q = reinterpret_cast<const u32x4_t*>(x + (g < nb ? g : g_cur) * (int64_t)block + (int64_t)li * kV);
        pf0 = __builtin_nontemporal_load(q);
        pf1 = __builtin_nontemporal_load(q + 1);
    };
    auto prefetch = [&](int64_t t, int64_t g_cur) __attribute__((always_inline)) {
        if (t >= nwork) return;
        prefetch_load(t, g_cur);
    };
    // the grid never exceeds the tiles, so first < nwork: no branch around these loads
    if constexpr (kPrefetch) prefetch_load(first, 0);
    {
        u32x4_t* dst4 = reinterpret_cast<u32x4_t*>(lut);
#pragma unroll
        for (int c = 0; c < kCopy; ++c) {
            const int i = (int)threadIdx.x + c * NTH;
            if (i < nw4) dst4[i] = cp[c];
        }
    }
    if (kQsLds && threadIdx.x < lpb * QSL) qsl[threadIdx.x] = qsv;
    __syncthreads();

    for (int64_t tile = first; tile < nwork; tile += stride) {
        int64_t gb;
        if (causal_t) {
            const int64_t m = tile / per_mat;
            const int64_t r = tile - m * per_mat;
            int64_t k = 0;
            while (8 * (k + 1) * (k + 2) <= r) ++k;
            const int64_t r2 = r - 8 * k * (k + 1);
            const int64_t rg = r2 / (k + 1), cb = r2 - rg * (k + 1);
            gb = (m * causal_t + 128 * k + 8 * rg + bw) * nbt + cb;
        } else {
            gb = tile * blocks_per_wg + (threadIdx.x / lpb);
        }
        const bool valid = gb < nb;
        const int64_t off = (valid ? gb : 0) * (int64_t)block + (int64_t)li * kV;

        // load 16 elements; the block max of |x| over the raw 16-bit patterns
        uint32_t w[8];
        if constexpr (kPrefetch) {
            // a lane past the end keeps the data it loaded: its block is never stored and
            // its lanes read only their own block's table rows
            w[0] = pf0.x; w[1] = pf0.y; w[2] = pf0.z; w[3] = pf0.w;
            w[4] = pf1.x; w[5] = pf1.y; w[6] = pf1.z; w[7] = pf1.w;
            prefetch(tile + stride, valid ? gb : 0);
        } else if (valid) {
            if constexpr (kMem) {
                const u32x4_t* q = reinterpret_cast<const u32x4_t*>(x + off);
                const u32x4_t a = __builtin_nontemporal_load(q), b = __builtin_nontemporal_load(q + 1);
                w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w; w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
            } else {
                // the producing pass's 16 outputs, computed here instead of read back
                const u32x4_t* qa = reinterpret_cast<const u32x4_t*>(src.a + off);
                const u32x4_t a0 = __builtin_nontemporal_load(qa), a1 = __builtin_nontemporal_load(qa + 1);
                const int64_t row = off / cols;
                const u32x4_t* qb = reinterpret_cast<const u32x4_t*>(src.b + (SRC == kSrcRms ? off - row * cols : off));
                const u32x4_t b0 = qb[0], b1 = qb[1];
                const uint32_t aw[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
                const uint32_t bw[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
                const float r = SRC == kSrcRms ? src.rs[row] : 0.f;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    uint32_t o[2];
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const float av = T::load((typename T::storage)(aw[i] >> (16 * h)));
                        const float bv = T::load((typename T::storage)(bw[i] >> (16 * h)));
                        o[h] = store_t<T>(SRC == kSrcRms ? rms_apply_one<T>(av, r, bv) : silu_mul_one<T>(av, bv));
                    }
                    w[i] = o[0] | (o[1] << 16);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) w[i] = 0u;
        }
        // packed 16-bit maxima (v_pk_max_u16) of the sign-cleared patterns, then the two halves
        typedef uint16_t u16x2_t __attribute__((ext_vector_type(2)));
        u16x2_t mp = __builtin_bit_cast(u16x2_t, w[0] & 0x7fff7fffu);
#pragma unroll
        for (int i = 1; i < 8; ++i) mp = __builtin_elementwise_max(mp, __builtin_bit_cast(u16x2_t, w[i] & 0x7fff7fffu));
        uint32_t m2 = mp.x > mp.y ? (uint32_t)mp.x : (uint32_t)mp.y;
        m2 = max8_dpp(m2);
        const float amax = T::load((typename T::storage)m2);
        float xa[kV];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            xa[2 * i] = fabsf(T::load((typename T::storage)(w[i] & 0xffffu)));
            xa[2 * i + 1] = fabsf(T::load((typename T::storage)(w[i] >> 16)));
        }

        float l1[S];
#pragma unroll
        for (int s = 0; s < S; ++s) {
            // R_T(amax * R32(1/em)) = R_T(amax / em) for quotients in T's normal range;
            // below it both clamp to 2^-14 (exhaustive CPU check over every T value)
            const float sr = T::round(amax * p.rem[s]);
            const float sc = __builtin_amdgcn_fmed3f(sr, 6.103515625e-05f, 61440.f);   // (v_med3 maps NaN to a bound)
            l1[s] = sr != sr ? sr : e5m3_scale<T>(sc, p.use_ceil);
        }

        // every block of this wave all zero (the masked half of causal attention weights):
        // the reference's result is +0 everywhere, level 0, the first L2 candidate and
        // scheme, and the L1 scale of a zero maximum computed above
        if (!__builtin_amdgcn_ballot_w64(m2 != 0u)) {
            if (valid) {
                float zero[kV];
#pragma unroll
                for (int i = 0; i < kV; ++i) zero[i] = 0.f;
                store16<T>(y + off, zero);
                if (codes) {
                    if constexpr (M == 1) *reinterpret_cast<uint2*>(codes + off / 2) = make_uint2(0u, 0u);
                    else *reinterpret_cast<uint4*>(codes + off) = make_uint4(0u, 0u, 0u, 0u);
                }
                if (li == 0) {
                    if (l1_out) l1_out[gb] = T::store(l1[0]);
                    if (sch_out) sch_out[gb] = 0;
                }
                if (l2i_out) {
                    constexpr int nsub_blk = block / L2B;
                    if (L2B <= kV) {
#pragma unroll
                        for (int sb = 0; sb < NSUBL; ++sb) l2i_out[gb * nsub_blk + (li * kV) / L2B + sb] = 0;
                    } else if ((li % LPS) == 0) {
                        l2i_out[gb * nsub_blk + (li * kV) / L2B] = 0;
                    }
                }
            }
            continue;
        }

        // magnitudes R_T(R_T(level * l2_j) * l1_s) of this block
        float qs[S][kFastJ][CPL];
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int j = 0; j < kFastJ; ++j)
#pragma unroll
                for (int k = 0; k < CPL; ++k) qs[s][j][k] = kQsLds ? qsl[li * QSL + (s * kFastJ + j) * CPL + k] : qreg[s][j][k];
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int j = 0; j < kFastJ; ++j)
#pragma unroll
                for (int k = 0; k < CPL; ++k) {
                    const int c = li + k * lpb;
                    if (c < L) {
                        const DT d = (DT)T::round(qs[s][j][k] * l1[s]);
                        DT* r = dwave + ((s * kFastJ + j) * bpw + bw) * ROW;
                        r[c] = d;
                        r[L + c] = -d;
                    }
                }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        h2_t xp[kV / 2];
        if constexpr (T::dt == kF16) {
#pragma unroll
            for (int i = 0; i < 8; ++i) xp[i] = __builtin_bit_cast(h2_t, w[i] & 0x7fff7fffu);
        }
        uint32_t ent[S][kV];
        // keys of t = R_T(|x| / l1): T's bit pattern shifted left by KSH (bf16: the
        // float bits of t, as BF16::round leaves them); non-negative, so ordered as integers
        constexpr int KSH = T::dt == kBF16 ? 16 : 0;
        uint32_t tb[S][kV];
        int jsel[S][NSUBL];
        uint32_t yws[S][8], cws[S][4];   // per scheme: output pairs and byte codes
        float errs[S];
        bool slow[S];
        float rl1v[S];
#pragma unroll
        for (int s = 0; s < S; ++s) {
            float rl1;   // l1 is an E5M3 value (or NaN): one v_rcp_f32 where the table build found it exact
            if (rcp_exact) {
                rl1 = __builtin_amdgcn_rcpf(l1[s]);
            } else {
                asm volatile("");   // a real (uniform) branch: keeps the division from being speculated
                rl1 = 1.0f / l1[s];
            }
            rl1v[s] = rl1;
            float qmin = xa[0] * rl1;
#pragma unroll
            for (int i = 0; i < kV; ++i) {
                const float q = xa[i] * rl1;
                qmin = fminf(qmin, q);
                tb[s][i] = key_of<T>(T::round(q));
            }
            slow[s] = qmin < tiny;
            if (slow[s]) {   // quotients in T's subnormal range can be exact ties: divide
#pragma unroll
                for (int i = 0; i < kV; ++i)
                    if (xa[i] * rl1 < tiny) tb[s][i] = key_of<T>(T::round(xa[i] / l1[s]));
            }
#pragma unroll
            for (int i = 0; i < kV; ++i) {
                int k;   // clamp to [-1, n] in one v_med3_i32; word k + 1 (0 and n + 1 are the sentinels)
                asm("v_med3_i32 %0, %1, -1, %2" : "=v"(k) : "v"((int)(tb[s][i] >> KSH) - (int)p.lo_bits), "s"(p.n));
                ent[s][i] = lut[s * per + k + 1];
            }
            float best[NSUBL];
#pragma unroll
            for (int j = 0; j < kFastJ; ++j) {
                if (j >= p.J) break;
                const char* rowb = drow0 + ((s * kFastJ + j) * bpw) * ROW * sizeof(DT);
#pragma unroll
                for (int sb = 0; sb < NSUBL; ++sb) {
                    // the squares are >= +0, so starting from the first one equals torch's 0 + ...
                    float acc;
#pragma unroll
                    for (int i = sb * SUBN; i < (sb + 1) * SUBN; i += 2) {
                        const DT d0 = *reinterpret_cast<const DT*>(rowb + ((ent[s][i] >> (8 * j)) & 0xffu));
                        const DT d1 = *reinterpret_cast<const DT*>(rowb + ((ent[s][i + 1] >> (8 * j)) & 0xffu));
                        if constexpr (T::dt == kF16) {
                            // R16(|x| - d) and R16(e^2) are single correctly rounded fp16 ops
                            const h2_t e = xp[i / 2] - (h2_t){d0, d1};
                            h2_t q = e * e;
                            asm("" : "+v"(q));
                            // acc + (float)q.x, acc + (float)q.y, each one v_fma_mix_f32
                            // (q * 1.0 + acc: the product is exact, so one fp32 rounding of
                            // the sum, as v_add_f32 after a conversion)
                            if (i == sb * SUBN) acc = (float)q.x;
                            else asm("v_fma_mix_f32 %0, %1, 1.0, %0 op_sel_hi:[1,0,0]" : "+v"(acc) : "v"(q));
                            asm("v_fma_mix_f32 %0, %1, 1.0, %0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "+v"(acc) : "v"(q));
                        } else {
                            float e0, e1, q0, q1;
                            round2<T>(xa[i] - (float)d0, xa[i + 1] - (float)d1, e0, e1);
                            round2<T>(e0 * e0, e1 * e1, q0, q1);
                            acc = i == sb * SUBN ? q0 : acc + q0;
                            acc += q1;
                        }
                    }
                    if constexpr (LPS == 2) {
                        // the lane pair's two partial sums: a DPP swap within the pair
                        // (quad_perm 1,0,3,2) and one add, the same bits in both lanes since
                        // a + b == b + a
                        const float o = __int_as_float(
                            __builtin_amdgcn_mov_dpp(__float_as_int(acc), 0xb1, 0xf, 0xf, true));
                        acc = acc + o;
                    } else if constexpr (LPS > 1) {
                        const int first = lane - (li % LPS);
                        float tot = __shfl(acc, first, 64);
                        for (int k2 = 1; k2 < LPS; ++k2) tot += __shfl(acc, first + k2, 64);
                        acc = tot;
                    }
                    const float sse = T::round(acc);
                    if (j == 0 || better(sse, best[sb])) {
                        best[sb] = sse;
                        jsel[s][sb] = j;
                    }
                }
            }
            // The selected candidate's level-word bytes (level times the entry size) of 4
            // elements in one register (v_perm_b32 picks byte j of two words at a time), and
            // the signs of x as byte masks (v_perm selectors 8-11 replicate bits 15, 31, 47
            // and 63 of its two input words: the signs of 4 packed 16-bit elements).
            constexpr int ES = (int)sizeof(DT);
            constexpr uint32_t kNeg = (uint32_t)(L * ES) * 0x01010101u;     // byte offset of -d in a row
            constexpr uint32_t kCodeSign = (1u << (M + 2)) * 0x01010101u;   // sign bit of a byte code
            uint32_t pb[4], xm[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const uint32_t j = (uint32_t)jsel[s][(4 * g) / SUBN];
                const uint32_t sel = j | ((j + 4u) << 8) | 0x0c0c0000u;   // byte j of the low word, then of the high word
                const uint32_t lo = __builtin_amdgcn_perm(ent[s][4 * g + 1], ent[s][4 * g], sel);
                const uint32_t hi = __builtin_amdgcn_perm(ent[s][4 * g + 3], ent[s][4 * g + 2], sel);
                pb[g] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
                xm[g] = __builtin_amdgcn_perm(w[2 * g + 1], w[2 * g], 0x0b0a0908u);
            }
            // The output keeps the sign of x unless u = R_T(t / l2_j) is 0 (then +0 and a
            // positive code), which needs t < z_j: a quotient below T's normal range, which
            // the check above flags (x = +-0 included).
            if (slow[s]) {
#pragma unroll
                for (int i = 0; i < kV; ++i) {
                    const int j = jsel[s][i / SUBN];
                    float zz = z[s][0];
#pragma unroll
                    for (int jj = 1; jj < kFastJ; ++jj) zz = j == jj ? z[s][jj] : zz;
                    // recomputed, not taken from the keys above: those die after the table index
                    uint32_t wv = w[i / 2];
                    asm("" : "+v"(wv));
                    const float a = fabsf(T::load((typename T::storage)(wv >> (16 * (i % 2)))));
                    const float q = a * rl1v[s];
                    const float t = q < tiny ? T::round(a / l1[s]) : T::round(q);
                    if (!(key_of<T>(t) >= key_of<T>(zz))) xm[i / 4] &= ~(0xffu << (8 * (i % 4)));
                }
            }
            // signed magnitudes: row of the selected candidate, byte offset plus L * ES if negative
            const char* rsel[NSUBL];
#pragma unroll
            for (int sb = 0; sb < NSUBL; ++sb) rsel[sb] = drow0 + ((s * kFastJ + jsel[s][sb]) * bpw) * ROW * ES;
            uint32_t ps[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) ps[g] = (xm[g] & kNeg) | pb[g];
            DT m[kV];
#pragma unroll
            for (int i = 0; i < kV; ++i)
                m[i] = *reinterpret_cast<const DT*>(rsel[i / SUBN] + ((ps[i / 4] >> (8 * (i % 4))) & 0xffu));
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                if constexpr (T::dt == kBF16) {   // the high halves: the values are bf16 already
                    yws[s][k] = __builtin_amdgcn_perm(f2bits((float)m[2 * k + 1]), f2bits((float)m[2 * k]), 0x07060302u);
                } else {
                    yws[s][k] = __builtin_bit_cast(uint32_t, (h2_t){(_Float16)m[2 * k], (_Float16)m[2 * k + 1]});
                }
            }
            // byte codes: level | sign << (M + 2)
#pragma unroll
            for (int g = 0; g < 4; ++g) cws[s][g] = (pb[g] / (uint32_t)ES) | (xm[g] & kCodeSign);
            if constexpr (S == 2) {
                // the scheme's block error: R_T(|x| - d) squared and rounded, summed over the
                // block in torch's order (|m| = d: the sign never changes the square)
                float sq[kV];
#pragma unroll
                for (int i = 0; i < kV; i += 2) {
                    if constexpr (T::dt == kF16) {
                        // single correctly rounded fp16 ops, as in the candidate search
                        const h2_t e = xp[i / 2] - __builtin_bit_cast(h2_t, yws[s][i / 2] & 0x7fff7fffu);
                        h2_t q = e * e;
                        asm("" : "+v"(q));
                        sq[i] = (float)q.x;
                        sq[i + 1] = (float)q.y;
                    } else {
                        float e0, e1;
                        round2<T>(xa[i] - fabsf((float)m[i]), xa[i + 1] - fabsf((float)m[i + 1]), e0, e1);
                        round2<T>(e0 * e0, e1 * e1, sq[i], sq[i + 1]);
                    }
                }
                errs[s] = T::round(block_row_sum8(sq, li));
            }
        }

        int sstar = 0;
        // Mix: the scheme with the smaller block error (the first on a tie), the same
        // value in the block's 8 lanes
        if constexpr (S == 2) sstar = better(errs[1], errs[0]) ? 1 : 0;
        uint32_t yw[8], cw[4];
#pragma unroll
        for (int k = 0; k < 8; ++k) yw[k] = (S == 2 && sstar) ? yws[S - 1][k] : yws[0][k];
#pragma unroll
        for (int g = 0; g < 4; ++g) cw[g] = (S == 2 && sstar) ? cws[S - 1][g] : cws[0][g];
        if (valid) {
            u32x4_t* q = reinterpret_cast<u32x4_t*>(y + off);
            __builtin_nontemporal_store((u32x4_t){yw[0], yw[1], yw[2], yw[3]}, q);
            __builtin_nontemporal_store((u32x4_t){yw[4], yw[5], yw[6], yw[7]}, q + 1);
            if (codes) {
                if constexpr (M == 1) {
                    // 4-bit codes, element 2i in the low nibble of byte i: bytes 0 and 2 of
                    // c | c >> 4 hold the nibble pairs of a word's 4 byte codes
                    uint32_t t[4];
#pragma unroll
                    for (int g = 0; g < 4; ++g) t[g] = cw[g] | (cw[g] >> 4);
                    *reinterpret_cast<uint2*>(codes + off / 2) =
                        make_uint2(__builtin_amdgcn_perm(t[1], t[0], 0x06040200u),
                                   __builtin_amdgcn_perm(t[3], t[2], 0x06040200u));
                } else {
                    *reinterpret_cast<uint4*>(codes + off) = make_uint4(cw[0], cw[1], cw[2], cw[3]);
                }
            }
        }
        if (valid) {
            if (li == 0) {
                if (l1_out) l1_out[gb] = T::store((S == 2 && sstar) ? l1[S - 1] : l1[0]);
                if (sch_out) sch_out[gb] = (uint8_t)sstar;
            }
            if (l2i_out) {
                constexpr int nsub_blk = block / L2B;
                const int s = (S == 2 && sstar) ? S - 1 : 0;
                if (L2B <= kV) {
#pragma unroll
                    for (int sb = 0; sb < NSUBL; ++sb)
                        l2i_out[gb * nsub_blk + (li * kV) / L2B + sb] = (uint8_t)jsel[s][sb];
                } else if ((li % LPS) == 0) {
                    l2i_out[gb * nsub_blk + (li * kV) / L2B] = (uint8_t)jsel[s][0];
                }
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
    }
}

// ---------------------------------------------------------------------------
// host side: table cache and dispatch
// ---------------------------------------------------------------------------
namespace {

struct LutKey {
    int dtype, mbit, scheme, l2_sc_bit, fused;
    bool operator==(const LutKey& o) const {
        return dtype == o.dtype && mbit == o.mbit && scheme == o.scheme && l2_sc_bit == o.l2_sc_bit &&
               fused == o.fused;
    }
};

constexpr int kMaxDevices = 64;
std::mutex g_mu;
LutKey g_keys[kMaxDevices][kLutSlots];
int g_state[kMaxDevices][kLutSlots];    // 0 empty, 1 ready, -1 unusable
int g_next[kMaxDevices];
int g_cus[kMaxDevices];

template <class T, int M>
int build_slot(int slot, const FastParams& p, hipStream_t st) {
    hipLaunchKernelGGL((build_lut_kernel<T, M>), dim3(64), dim3(256), 0, st, slot, p);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return hbq_fail(HBQ_ERR_HIP, "HBQ level table build failed: %s", hipGetErrorString(e));
    int status = -1;
    e = hipMemcpyFromSymbol(&status, HIP_SYMBOL(g_lut_status), sizeof(int), sizeof(int) * slot,
                            hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hbq_fail(HBQ_ERR_HIP, "HBQ level table status read failed: %s", hipGetErrorString(e));
    return status;   // 0 ready, > 0 the table shape does not fit this configuration
}

template <class T, int M, int L2B, int S, int SRC = kSrcX>
int launch_fast(const void* x, void* y, void* l1, void* l2i, void* sch, void* codes, int64_t nb, int64_t causal_t,
                int slot, const FastParams& p, int dev, hipStream_t st, const FastSrc& src = FastSrc{}, int64_t cols = 0) {
    constexpr int lpb_log2 = 3;
    constexpr int NTH = fast_threads<T, M, S>();
    using St = typename T::storage;
    constexpr int CPL = ((1 << (M + 2)) + 7) / 8;   // the level constants in LDS: two-scheme kernels
    const size_t lds = (S == 2 ? (size_t)(S * (p.n + 2) + 3) / 4 * 16 + (size_t)8 * S * kFastJ * CPL * 4
                               : (size_t)S * (p.n + 2) * 4) +
                       (size_t)(NTH >> lpb_log2) * S * kFastJ * fast_row<T, M>() * sizeof(DTabT<T>);
    if (lds > 160 * 1024) return 0;
    if constexpr (SRC == kSrcX) {
        if (causal_t) return launch_fast<T, M, L2B, S, kSrcXCausal>(x, y, l1, l2i, sch, codes, nb, causal_t, slot, p, dev, st);
    }
    auto kern = hbq_fast_kernel<T, M, L2B, S, SRC>;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, NTH, lds) != hipSuccess || per_cu <= 0)
        return 0;
    const int64_t blocks_per_wg = NTH >> lpb_log2;
    int64_t ntiles = (nb + blocks_per_wg - 1) / blocks_per_wg;
    if (causal_t) {   // wave units on or below the diagonal, NTH / 64 a workgroup
        const int64_t nbt = causal_t / 128, units = nb / (causal_t * nbt) * 8 * nbt * (nbt + 1);
        ntiles = (units + NTH / 64 - 1) / (NTH / 64);
    }
    // as many rounds as the resident workgroups need, with the tiles spread evenly over
    // them (a last round with few tiles would leave most of the chip idle)
    const int64_t resident = (int64_t)g_cus[dev] * per_cu;
    const int64_t rounds = (ntiles + resident - 1) / resident;
    const int64_t grid = (ntiles + rounds - 1) / rounds;
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(NTH), lds, st, (const St*)x, (St*)y, (St*)l1,
                       (uint8_t*)l2i, (uint8_t*)sch, (uint8_t*)codes, nb, causal_t, slot, p, src, cols);
    return 1;
}

template <class T, int M>
int fast_by_shape(int l2b, int S, const void* x, void* y, void* l1, void* l2i, void* sch, void* codes, int64_t cols,
                  int block, int lpb_log2, int64_t nb, int64_t causal_t, int slot, const FastParams& p, int dev,
                  hipStream_t st) {
#define FAST_CASE(LB, SS)                                                                                   \
    if (l2b == LB && S == SS)                                                                               \
        return launch_fast<T, M, LB, SS>(x, y, l1, l2i, sch, codes, nb, causal_t, slot, p, dev, st);
    FAST_CASE(8, 1) FAST_CASE(8, 2) FAST_CASE(16, 1) FAST_CASE(16, 2) FAST_CASE(32, 1) FAST_CASE(32, 2)
#undef FAST_CASE
    return 0;
}

}  // namespace
}  // namespace hbq

using namespace hbq;

// Configuration checks, kernel parameters and the per-device level table of the table
// kernel: 1 ready (p, slot, dev set), 0 not for this kernel, < 0 a HIP error.
static int fast_setup(FastParams& p, int& slot, int& dev, int dtype, int block, int mbit, int l2b, int l2_sc_bit,
                      int scheme, const HbqParams& hp, hipStream_t st) {
    if (dtype != kF16 && dtype != kBF16) return 0;
    if (mbit < 1 || mbit > 3 || hp.J > kFastJ) return 0;
    if (l2b != 8 && l2b != 16 && l2b != 32) return 0;
    if (block != 128 || block % l2b) return 0;
    const int S = scheme == 7 ? 2 : 1;

    // table range [2^lo, 2^hi): below 2^-(m+2) every candidate rounds to level 0 (l2 >= 1);
    // at or above 8 * max(l2) every candidate saturates
    float l2max = 1.f;
    for (int s = 0; s < S; ++s)
        for (int j = 0; j < hp.J; ++j) l2max = hp.l2[j][s] > l2max ? hp.l2[j][s] : l2max;
    int hi = 3;
    while ((float)(1 << (hi - 3)) < l2max) ++hi;
    const int lo = -(mbit + 2);
    if (hi - lo > kLutMaxBinades) return 0;
    p = FastParams{};
    p.S = S;
    p.J = hp.J;
    p.L = 1 << (mbit + 2);
    const int mbits_T = dtype == kF16 ? 10 : 7;
    const int bias = dtype == kF16 ? 15 : 127;
    p.n = (hi - lo) << mbits_T;
    p.lo_bits = (uint32_t)(bias + lo) << mbits_T;
    for (int j = 0; j < kFastJ; ++j)
        for (int s = 0; s < 2; ++s) p.l2[j][s] = j < hp.J ? hp.l2[j][s] : 1.f;
    p.em[0] = hp.em[0];
    p.em[1] = hp.em[S - 1];
    p.rem[0] = 1.0f / p.em[0];
    p.rem[1] = 1.0f / p.em[1];
    p.use_ceil = hp.sf.use_ceil;
    p.fused = hp.fused;
    // the kernel quantizes the L1 scale to E5M3 without subnormals
    if (hp.sf.allow_sub || hp.sf.emax != 15.f || hp.sf.mshift != 8.f || hp.sf.emin != -14.f) return 0;

    dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
    slot = -1;
    std::lock_guard<std::mutex> g(g_mu);
    if (g_cus[dev] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            return 0;
        g_cus[dev] = cus;
    }
    const LutKey key{dtype, mbit, scheme, l2_sc_bit, hp.fused};
    for (int i = 0; i < kLutSlots; ++i)
        if (g_state[dev][i] != 0 && g_keys[dev][i] == key) slot = i;
    if (slot >= 0 && g_state[dev][slot] < 0) return 0;
    if (slot < 0) {
        slot = g_next[dev];
        g_next[dev] = (g_next[dev] + 1) % kLutSlots;
        g_keys[dev][slot] = key;
        int rc;
        if (dtype == kF16)
            rc = mbit == 1 ? build_slot<F16, 1>(slot, p, st) : mbit == 2 ? build_slot<F16, 2>(slot, p, st)
                                                                           : build_slot<F16, 3>(slot, p, st);
        else
            rc = mbit == 1 ? build_slot<BF16, 1>(slot, p, st) : mbit == 2 ? build_slot<BF16, 2>(slot, p, st)
                                                                            : build_slot<BF16, 3>(slot, p, st);
        if (rc < 0 || rc == HBQ_ERR_HIP) {
            g_state[dev][slot] = 0;
            return -HBQ_ERR_HIP;
        }
        g_state[dev][slot] = rc == 0 ? 1 : -1;
        if (rc != 0) return 0;
    }
    return 1;
}

int hbq_fast_try(const void* x, void* y, void* l1, void* l2i, void* sch, void* codes, int64_t rows, int64_t cols,
                 int dtype, int block, int mbit, int l2b, int l2_sc_bit, int scheme, const HbqParams& hp,
                 hipStream_t st, int64_t causal_t) {
    if (block != 128 || cols % block || ((uintptr_t)x % 16) || ((uintptr_t)y % 16) ||
        (codes && ((uintptr_t)codes % 16)))
        return 0;
    FastParams p;
    int slot = -1, dev = 0;
    const int rs = fast_setup(p, slot, dev, dtype, block, mbit, l2b, l2_sc_bit, scheme, hp, st);
    if (rs <= 0) return rs;
    const int S = p.S;
    const int64_t nb = rows * (cols / block);
    if (nb == 0) return 1;
    const int lpb_log2 = 3;
    int done;
#define FAST_T(TT)                                                                                              \
    (mbit == 1 ? fast_by_shape<TT, 1>(l2b, S, x, y, l1, l2i, sch, codes, cols, block, lpb_log2, nb, causal_t, slot, p, dev, st) \
     : mbit == 2 ? fast_by_shape<TT, 2>(l2b, S, x, y, l1, l2i, sch, codes, cols, block, lpb_log2, nb, causal_t, slot, p, dev, st) \
                 : fast_by_shape<TT, 3>(l2b, S, x, y, l1, l2i, sch, codes, cols, block, lpb_log2, nb, causal_t, slot, p, dev, st))
    done = dtype == kF16 ? FAST_T(F16) : FAST_T(BF16);
#undef FAST_T
    return done;
}

namespace {
template <class T, int SRC>
int launch_src(int l2b, void* y, int64_t nb, int slot, const FastParams& p, int dev, hipStream_t st,
               const FastSrc& src, int64_t cols) {
    switch (l2b) {
        case 8: return launch_fast<T, 2, 8, 1, SRC>(nullptr, y, nullptr, nullptr, nullptr, nullptr, nb, 0, slot, p, dev, st, src, cols);
        case 16: return launch_fast<T, 2, 16, 1, SRC>(nullptr, y, nullptr, nullptr, nullptr, nullptr, nb, 0, slot, p, dev, st, src, cols);
        case 32: return launch_fast<T, 2, 32, 1, SRC>(nullptr, y, nullptr, nullptr, nullptr, nullptr, nb, 0, slot, p, dev, st, src, cols);
    }
    return 0;
}
}  // namespace

int hbq_fast_try_src(const FastSrc& src, void* y, int64_t rows, int64_t cols, int dtype, int block, int mbit,
                     int l2b, int l2_sc_bit, int scheme, const HbqParams& hp, hipStream_t st) {
    // the activation formats only (E2M2 elements, one scheme): the kernels instantiated here
    if (mbit != 2 || scheme == 7 || (src.kind != kSrcRms && src.kind != kSrcSilu)) return 0;
    if (block != 128 || cols % block || ((uintptr_t)y % 16) || ((uintptr_t)src.a % 16) || ((uintptr_t)src.b % 16))
        return 0;
    FastParams p;
    int slot = -1, dev = 0;
    const int rs = fast_setup(p, slot, dev, dtype, block, mbit, l2b, l2_sc_bit, scheme, hp, st);
    if (rs <= 0) return rs;
    const int64_t nb = rows * (cols / block);
    if (nb == 0) return 1;
    if (dtype == kF16)
        return src.kind == kSrcRms ? launch_src<F16, kSrcRms>(l2b, y, nb, slot, p, dev, st, src, cols)
                                   : launch_src<F16, kSrcSilu>(l2b, y, nb, slot, p, dev, st, src, cols);
    return src.kind == kSrcRms ? launch_src<BF16, kSrcRms>(l2b, y, nb, slot, p, dev, st, src, cols)
                               : launch_src<BF16, kSrcSilu>(l2b, y, nb, slot, p, dev, st, src, cols);
}
