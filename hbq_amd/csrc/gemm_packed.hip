// GEMM on packed HBQ weights for decode-sized M (<= 32 rows): C[M,N] = A[M,K]
// x dequant(W)[N,K]^T, the weight read as packed E2M1 codes and scale bytes
// (pack.hip's format) and decoded in registers straight into the MFMA operand.
//
// A workgroup per 32 output columns, all M rows (padded to 32 with zero rows).
// A group of 8 consecutive codes of a weight row (one 32-bit load) decodes to the
// fp16 values the unpack kernel writes:
//   the level bits l placed at fp16 bits [11:9] are the fp16 value l * 2^-14
//   (exponent field 0 included); one v_pk_mul_f16 by R16(l2[j][s] * 2^14) gives
//   R16(level * l2) (an exact product rounded once), one by the E5M3 scale
//   (whose byte is fp16 bits [14:7]) gives R16(R16(level * l2) * l1), and the
//   code's sign is or-ed in (src/quantizer.py:790-796).
// The MFMA sequence per output element (v_mfma_f32_32x32x16_f16 in ascending K
// steps, zero C at each group start) and the group folds are those of the
// 128x128 and 256-row kernels, so C has the same bits as the GEMM on the
// unpacked weight.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

#include "gemm_common.h"
#include "hbq_capi_internal.h"
#include "quant_common.h"

namespace hbq_gemm {
namespace {

constexpr int kWaves = 4;   // waves per workgroup: one runs the MFMAs, three decode

struct PackedW {
    const uint8_t* codes;   // [N, K / 2]
    const uint8_t* l1;      // [N, K / 128]
    const uint8_t* l2;      // [N, l2_row] or null
    const uint8_t* sch;     // [N, sch_row] (Mix) or null
    int64_t l2_row, sch_row;
    int l2b, l2bits, S;
    uint32_t l2x[4][2];     // fp16 R16(l2[j][s] * 2^14) in both halves
};


// Workgroup barrier for LDS traffic only: this wave's LDS accesses are complete,
// while its global loads stay in flight (__syncthreads would also wait for those,
// which are issued chunks ahead of their use).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// f(integral_constant<int, D>) for D = 0, 1, ... in order, with D a compile-time constant
template <class F, int... D>
__device__ __forceinline__ void for_each_index(F&& f, std::integer_sequence<int, D...>) {
    (f(std::integral_constant<int, D>{}), ...);
}

// The row window [kb, kb + 128) of a chunk: the decoded fp16 values of one group of
// 8 codes of weight row n (E2M1), as described at the top of the file.
struct DecodeIn {
    uint32_t cw;     // 8 codes
    uint32_t l1x;    // E5M3 scale as an fp16 pair
    uint32_t l2x;    // R16(l2[j][s] * 2^14) as an fp16 pair
};

__device__ __forceinline__ u32x4 decode8(const DecodeIn& d) {
    const uint32_t x0 = d.cw & 0x0F0F0F0Fu, x1 = (d.cw >> 4) & 0x0F0F0F0Fu;
    u32x4 bw;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        // (code of element 2p + 1) << 16 | code of element 2p
        const uint32_t hp = __builtin_amdgcn_perm(x1, x0, 0x0c000c00u | ((4u + p) << 16) | (uint32_t)p);
        const h2_t mag = __builtin_bit_cast(h2_t, (hp << 9) & 0x0E000E00u);
        const h2_t v = (mag * __builtin_bit_cast(h2_t, d.l2x)) * __builtin_bit_cast(h2_t, d.l1x);
        bw[p] = __builtin_bit_cast(uint32_t, v) | ((hp << 12) & 0x80008000u);
    }
    return bw;
}

// A workgroup of 4 waves owns 32 output columns (weight rows n0 .. n0 + 31) and all
// M rows.  K runs in chunks of 128 through a two-buffer LDS ring holding each
// chunk's decoded weights and A rows: waves 1..3 issue the global loads of a chunk
// kDepth chunks ahead (a register ring) and decode / copy chunk c + 1 into LDS
// while wave 0 runs the 8 MFMA steps of chunk c from LDS; one barrier per chunk.
// Wave 0 alone holds the accumulators, so the MFMA chain per output element is
// the single ascending chain of the other GEMM kernels.
constexpr int kRowPitch = 128 + 8;   // halfs; 272-byte rows keep the 16-byte operand reads conflict-free
constexpr int kGroups = 32 * 16;     // groups of 8 values per chunk (weights, and A rows)
constexpr int kDecLanes = 192;       // lanes of waves 1..3
constexpr int kGPL = (kGroups + kDecLanes - 1) / kDecLanes;   // groups per loading lane (3)
constexpr int kDepth = 2;            // chunks of global loads in flight per loading lane (K % (128 kDepth) == 0)

template <int MODE, int GN>
__global__ __launch_bounds__(64 * kWaves) void packed_gemm_kernel(const uint16_t* __restrict__ A, PackedW w,
                                                                  uint16_t* __restrict__ C, int M, int N, int K,
                                                                  int gk) {
    __shared__ __attribute__((aligned(16))) uint16_t Wd[2][32 * kRowPitch];
    __shared__ __attribute__((aligned(16))) uint16_t Ad[2][32 * kRowPitch];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n0 = blockIdx.x * 32;
    const int nchunks = K / 128;

    // ---- loading lanes (waves 1..3): global -> register ring -> LDS ----
    // The ring keeps the loaded words as they arrive: nothing in a fetch uses a loaded
    // value (a use inside the fetch would make it wait for the load), and every load is
    // unconditional (absent strings read a valid dummy byte), so the loads of kDepth
    // chunks stay in flight together.
    struct Raw {
        uint32_t cw;    // 8 codes
        uint32_t l1b;   // L1 byte
        uint32_t scb;   // scheme byte
        uint32_t l2b0, l2b1;   // the L2 bytes holding the group's index
    };
    __shared__ uint32_t l2x_lds[8];
    if (threadIdx.x < 8) l2x_lds[threadIdx.x] = w.l2x[threadIdx.x >> 1][threadIdx.x & 1];
    const int dl = threadIdx.x - 64;   // 0..191 on waves 1..3
    Raw ring[kDepth][kGPL];
    u32x4 aring[kDepth][kGPL];
    // this lane's groups: fixed row and column offset inside every chunk, so the
    // addresses are set up once and advance by a constant per chunk
    const uint8_t* pc[kGPL];      // codes
    const uint8_t* pl1[kGPL];     // L1 bytes
    const uint8_t* psc[kGPL];     // scheme bytes (row start)
    const uint8_t* pl2[kGPL];     // L2 bytes (row start)
    const uint16_t* pa[kGPL];     // A
    int l2pos[kGPL];              // bit position of the group's sub-block in chunk 0
    bool has_a[kGPL], valid[kGPL];
    const int bits_per_chunk = (128 / w.l2b) * w.l2bits;
    const int l2_last = w.l2 ? (int)w.l2_row - 1 : 0;
#pragma unroll
    for (int i = 0; i < kGPL; ++i) {
        const int g0 = dl + kDecLanes * i;
        valid[i] = dl >= 0 && g0 < kGroups;
        const int g = valid[i] ? g0 : 0;
        const int r = g >> 4, kofs = (g & 15) << 3;
        const int64_t n = n0 + r;
        pc[i] = w.codes + n * (K / 2) + (kofs >> 1);
        pl1[i] = w.l1 + n * (K / 128);
        psc[i] = w.sch ? w.sch + n * w.sch_row : pl1[i];     // absent strings: a valid dummy byte
        pl2[i] = w.l2 ? w.l2 + n * w.l2_row : pl1[i];
        has_a[i] = r < M;
        pa[i] = A + (int64_t)(has_a[i] ? r : 0) * K + kofs;
        l2pos[i] = w.l2bits ? (kofs / w.l2b) * w.l2bits : 0;
    }
    // branch-free: chunks past the end re-read the last one, groups past the end a valid one
    auto fetch = [&](int c, Raw (&f)[kGPL], u32x4 (&fa)[kGPL]) __attribute__((always_inline)) {
        c = c < nchunks ? c : nchunks - 1;
#pragma unroll
        for (int i = 0; i < kGPL; ++i) {
            f[i].cw = *reinterpret_cast<const uint32_t*>(pc[i] + c * 64);
            f[i].l1b = pl1[i][c];
            f[i].scb = psc[i][w.S == 2 ? (c >> 3) : 0];
            const int byte = w.l2bits ? (c * bits_per_chunk + l2pos[i]) >> 3 : 0;
            f[i].l2b0 = pl2[i][byte];
            f[i].l2b1 = pl2[i][byte + 1 < l2_last ? byte + 1 : l2_last];
            fa[i] = *reinterpret_cast<const u32x4*>(pa[i] + c * 128);
        }
    };
    auto store = [&](int c, int buf, const Raw (&f)[kGPL], const u32x4 (&fa)[kGPL]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < kGPL; ++i) {
            if (valid[i]) {
                const int g = dl + kDecLanes * i;
                const int sb = w.S == 2 ? (int)((f[i].scb >> (c & 7)) & 1u) : 0;
                const int pos = (c * bits_per_chunk + l2pos[i]) & 7;
                const uint32_t l2w = f[i].l2b0 | (f[i].l2b1 << 8);
                const int j = w.l2bits ? (int)((l2w >> pos) & ((1u << w.l2bits) - 1u)) : 0;
                DecodeIn d;
                d.cw = f[i].cw;
                d.l1x = f[i].l1b * 0x00800080u;
                d.l2x = l2x_lds[j * 2 + sb];
                const int off = (g >> 4) * kRowPitch + ((g & 15) << 3);
                *reinterpret_cast<u32x4*>(&Wd[buf][off]) = decode8(d);
                *reinterpret_cast<u32x4*>(&Ad[buf][off]) = has_a[i] ? fa[i] : (u32x4){0u, 0u, 0u, 0u};
            }
        }
    };

    // ---- MFMA lanes (wave 0) ----
    const int h = lane >> 5;
    const int m = lane & 31;
    f16v acc = {};
    h2_t H[8];
#pragma unroll
    for (int p = 0; p < 8; ++p) H[p] = (h2_t){(_Float16)0.f, (_Float16)0.f};
    const int gsteps = gk / 16;
    auto mfma_chunk = [&](int c) __attribute__((always_inline)) {
        const int buf = c & 1;
        const uint16_t* wrow = &Wd[buf][m * kRowPitch + 8 * h];   // weight row n0 + (lane % 32)
        const uint16_t* arow = &Ad[buf][m * kRowPitch + 8 * h];   // A row lane % 32
#pragma unroll
        for (int st = 0; st < 8; ++st) {
            const h8 bop = *reinterpret_cast<const h8*>(wrow + 16 * st);
            const h8 aop = *reinterpret_cast<const h8*>(arow + 16 * st);
            const int step = c * 8 + st;
            // a group's first MFMA adds to +0 (acc is reset after every fold)
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(bop, aop, acc, 0, 0, 0);
            if constexpr (MODE != kFp32) {
                if (step % gsteps == gsteps - 1) {
                    f16v accs[1][1] = {{acc}};
                    h2_t Hs[1][1][8];
#pragma unroll
                    for (int p = 0; p < 8; ++p) Hs[0][0][p] = H[p];
                    fold_all<MODE, GN>(accs, Hs);
#pragma unroll
                    for (int p = 0; p < 8; ++p) H[p] = Hs[0][0][p];
                    acc = (f16v){};
                }
            }
        }
    };

    __syncthreads();   // the L2 factor table
    if (wave > 0) {
#pragma unroll
        for (int d = 0; d < kDepth; ++d) fetch(d, ring[d], aring[d]);
        store(0, 0, ring[0], aring[0]);
        fetch(kDepth, ring[0], aring[0]);
    }
    lds_barrier();

    // chunk c + 1 sits in ring slot (c + 1) % kDepth; the loop is unrolled by kDepth with
    // compile-time slot indices (a fold expression: the body is too large for the unroller)
    auto one_chunk = [&](int c0, auto d_tag) __attribute__((always_inline)) {
        constexpr int D = decltype(d_tag)::value;
        const int c = c0 + D;   // nchunks is a multiple of kDepth
        if (wave > 0) {
            if (c + 1 < nchunks) {
                constexpr int SL = (D + 1) % kDepth;
                store(c + 1, (c + 1) & 1, ring[SL], aring[SL]);
                fetch(c + 1 + kDepth, ring[SL], aring[SL]);
            }
        } else {
            mfma_chunk(c);
        }
        lds_barrier();
    };
    for (int c0 = 0; c0 < nchunks; c0 += kDepth)
        for_each_index([&](auto d_tag) __attribute__((always_inline)) { one_chunk(c0, d_tag); },
                       std::make_integer_sequence<int, kDepth>{});
    if (wave > 0 || m >= M) return;
    // lane (m, h) holds columns n0 + 8 (r / 4) + 4 h + (r % 4) of row m
    uint16_t* crow = C + (int64_t)m * N + n0 + 4 * h;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        h2_t lo, hi;
        if constexpr (MODE == kFp32) {
            lo = cvt2(acc[4 * q], acc[4 * q + 1]);
            hi = cvt2(acc[4 * q + 2], acc[4 * q + 3]);
        } else {
            lo = H[2 * q];
            hi = H[2 * q + 1];
        }
        *reinterpret_cast<uint2*>(crow + 8 * q) =
            make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
    }
}

template <int MODE, int GN>
void launch(const void* A, const PackedW& w, void* C, int M, int N, int K, int gk, hipStream_t st) {
    const dim3 grid((unsigned)(N / 32));
    hipLaunchKernelGGL((packed_gemm_kernel<MODE, GN>), grid, dim3(64 * kWaves), 0, st, (const uint16_t*)A, w,
                       (uint16_t*)C, M, N, K, gk);
}

}  // namespace
}  // namespace hbq_gemm

using namespace hbq_gemm;

extern "C" {

int hbq_gemm_packed_w(const void* A, const void* pcodes, const void* pl1, const void* pl2, const void* pscheme,
                      void* C, int M, int N, int K, int block_size, int mbit, int l2_block_size, int l2_sc_bit,
                      int l2_scheme, int acc_mode, int group_k, int group_n, void* stream) {
    hbq_clear_error();
    if (M < 1 || M > 32) return hbq_fail(HBQ_ERR_UNSUPPORTED, "the packed-weight GEMM takes 1..32 rows, got %d", M);
    if (N < 32 || N % 32 || K < 128 * kDepth || K % (128 * kDepth))
        return hbq_fail(HBQ_ERR_UNSUPPORTED, "the packed-weight GEMM needs N %% 32 == 0 and K %% %d == 0", 128 * kDepth);
    if (block_size != 128 || mbit != 1)
        return hbq_fail(HBQ_ERR_UNSUPPORTED, "the packed-weight GEMM takes E2M1 codes in blocks of 128");
    if (l2_block_size != 8 && l2_block_size != 16 && l2_block_size != 32)
        return hbq_fail(HBQ_ERR_UNSUPPORTED, "l2_block_size must be 8, 16 or 32");
    if (l2_sc_bit < 0 || l2_sc_bit > 2) return hbq_fail(HBQ_ERR_UNSUPPORTED, "l2_sc_bit must be 0..2");
    if (!A || !pcodes || !pl1 || !C || (l2_sc_bit && !pl2) || (l2_scheme == 7 && !pscheme))
        return hbq_fail(HBQ_ERR_INVALID, "null pointer");
    if ((uintptr_t)A % 16 || (uintptr_t)pcodes % 4 || (uintptr_t)C % 8)
        return hbq_fail(HBQ_ERR_INVALID, "misaligned operand");
    hbq::HbqParams hp{};
    int S = 1;
    if (int rc = hbq::hbq_l2_table(hp, S, l2_sc_bit, l2_scheme, hbq::kF16)) return rc;
    PackedW w{};
    w.codes = (const uint8_t*)pcodes;
    w.l1 = (const uint8_t*)pl1;
    w.l2 = l2_sc_bit ? (const uint8_t*)pl2 : nullptr;
    w.sch = S == 2 ? (const uint8_t*)pscheme : nullptr;
    w.l2_row = ((int64_t)K / l2_block_size * l2_sc_bit + 7) / 8;
    w.sch_row = (K / 128 + 7) / 8;
    w.l2b = l2_block_size;
    w.l2bits = l2_sc_bit;
    w.S = S;
    for (int j = 0; j < 4; ++j)
        for (int s = 0; s < 2; ++s) {
            const float v = j < hp.J ? hp.l2[j][s] : 1.f;
            if (!(v * 16384.f <= 65504.f))
                return hbq_fail(HBQ_ERR_UNSUPPORTED, "L2 factors of 4 and above need the unpacked path");
            const uint16_t b = __builtin_bit_cast(uint16_t, (_Float16)(v * 16384.f));
            w.l2x[j][s] = (uint32_t)b * 0x00010001u;
        }
    hipStream_t st = (hipStream_t)stream;
    switch (acc_mode) {
        case 0: launch<kFp32, 4>(A, w, C, M, N, K, K, st); break;
        case 1:
            if (group_k != 16 && group_k != 32 && group_k != 64 && group_k != 128)
                return hbq_fail(HBQ_ERR_INVALID, "group_k must be one of {16,32,64,128}");
            if (K % group_k) return hbq_fail(HBQ_ERR_INVALID, "K must be divisible by group_k");
            launch<kGrouped, 4>(A, w, C, M, N, K, group_k, st);
            break;
        case 2:
        case 3: {
            if (group_k != 64 && group_k != 128 && group_k != 256)
                return hbq_fail(HBQ_ERR_INVALID, "group_k must be one of {64,128,256}");
            if (K % group_k) return hbq_fail(HBQ_ERR_INVALID, "K must be divisible by group_k");
            if (group_n != 4 && group_n != 8 && group_n != 16 && group_n != 32)
                return hbq_fail(HBQ_ERR_INVALID, "group_n must be one of {4,8,16,32}");
#define PW_GN(MD)                                                          \
    switch (group_n) {                                                     \
        case 4: launch<MD, 4>(A, w, C, M, N, K, group_k, st); break;       \
        case 8: launch<MD, 8>(A, w, C, M, N, K, group_k, st); break;       \
        case 16: launch<MD, 16>(A, w, C, M, N, K, group_k, st); break;     \
        default: launch<MD, 32>(A, w, C, M, N, K, group_k, st); break;     \
    }
            if (acc_mode == 2) { PW_GN(kInt8) } else { PW_GN(kFp8) }
#undef PW_GN
            break;
        }
        default: return hbq_fail(HBQ_ERR_INVALID, "bad accumulation mode %d", acc_mode);
    }
    return hbq_check_launch("hbq_gemm_packed_w");
}

}  // extern "C"
