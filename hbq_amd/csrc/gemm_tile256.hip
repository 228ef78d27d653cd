// 256x256-tile block-quant GEMM for gfx950, C[M,N] = A[M,K] W[N,K]^T (fp16).
//
// One 512-thread workgroup (8 waves) per 256x256 output tile; each wave owns
// a 128 (rows) x 64 (columns) sub-tile: 4 x 2 blocks of
// v_mfma_f32_32x32x16_f16 with the operands swapped (see gemm_common.h), so a
// psum group of up to 32 columns of one row lives in one lane pair.
//
// Operand staging: 64-wide K slices of A and W go straight from global memory
// into LDS with buffer_load_dwordx4 ... lds (no register staging), double
// buffered (2 x 64 KB).  A row of a slice is 128 B = 8 chunks of 16 B, stored
// in a swizzled order (swz_pos) that keeps the 16-byte operand reads of
// consecutive rows free of bank conflicts.
//
// Tile order: consecutive workgroups go round-robin to the 8 XCDs, so tile
// indices are first regrouped to give each XCD a contiguous range, then
// walked in 4-row-tile column bands: the tiles resident on one XCD share A
// rows and W rows in that XCD's L2.
//
// Group ends (group_k >= 64) fall on stage boundaries; group_k 16/32 (grouped
// accumulation only) fold inside a stage.  At the end the fp16 accumulators go
// through LDS to give full 128-byte row segments on the store.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "gemm_common.h"
#include "gemm_tile256.h"

namespace hbq_gemm {
namespace t256 {

constexpr int TM = 256, TK = 64, NT = 512;
constexpr int SLICE = TM * TK;   // halfs of one A slice (32 KB)

// chunk c of row r sits at chunk position c ^ (r % 8) ^ ((r / 8) % 2): any 8
// consecutive rows use 8 different positions, and any 16 consecutive rows 16
// different (row parity, position) pairs, so 16-byte reads of consecutive rows
// spread over all banks for a 128-byte as well as a 256-byte bank period
__device__ __forceinline__ int swz_pos(int row, int chunk) { return chunk ^ (row & 7) ^ ((row >> 3) & 1); }
__device__ __forceinline__ int swz(int row, int chunk) { return row * TK + 8 * swz_pos(row, chunk); }

// SMALLG: group_k < 64 (grouped accumulation with group_k 16 or 32, or group
// partials), GS = group_k / 16 steps per group; otherwise SPG = group_k / 64
// slices per group (K is a multiple of group_k).  TN: tile width, 256 (waves
// of 128 x 64) or 128 (waves of 64 x 64, for grids that 256-wide tiles would
// leave short of the compute units).
template <int MODE, int GN, bool SMALLG, int GS, int SPG, int TN>
__global__ __launch_bounds__(NT, 1) void kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ W,
                                                uint16_t* __restrict__ C, float* __restrict__ P, int M, int N, int K,
                                                int gk, int tiles_m, int tiles_n, int splits, int batches,
                                                int64_t sA, int64_t sW, int64_t sC, int wgroup, int64_t ldc) {
    constexpr int WSL = TN * TK;          // halfs of one W slice
    constexpr int NWN = TN / 64;          // waves across the tile's columns
    constexpr int WROWS = TM * NWN / 8;   // rows of one wave (128 or 64)
    constexpr int RB = WROWS / 32;        // 32-row blocks of one wave
    __shared__ __attribute__((aligned(1024))) uint16_t smem[2 * SLICE + 2 * WSL];
    uint16_t* const sA0 = smem;
    uint16_t* const sA1 = smem + SLICE;
    uint16_t* const sW0 = smem + 2 * SLICE;
    uint16_t* const sW1 = smem + 2 * SLICE + WSL;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    // ---- tile of this workgroup ----
    const int T = tiles_m * tiles_n;
    int u = blockIdx.x;
    // split K (fp32 accumulation): workgroups [s T, (s + 1) T) take the s-th of `splits`
    // equal K ranges and write their fp32 partial sums to P[s]
    int split = 0;
    if (MODE == kFp32 && splits > 1) {
        split = u / T;
        u -= split * T;
        A += (int64_t)split * (K / splits);
        W += (int64_t)split * (K / splits);
    } else if (batches > 1) {   // batched: workgroups [z T, (z + 1) T) take problem z
        const int z = u / T;
        u -= z * T;
        A += z * sA;
        W += (z / wgroup) * sW;   // problems z of one W group share W (grouped-query attention)
        C += z * sC;
    }
    if ((T & 7) == 0) u = (u & 7) * (T >> 3) + (u >> 3);
    const int band = 4 * tiles_n;
    const int first = (u / band) * 4;
    const int rows_in_band = min(tiles_m - first, 4);
    const int within = u % band;
    const int tm = first + within % rows_in_band;
    const int tn = within / rows_in_band;
    const int m0 = tm * TM, n0 = tn * TN;
    const int wm = (wave / NWN) * WROWS;   // wave's rows in the tile
    const int wn = (wave % NWN) * 64;      // wave's columns in the tile

    // ---- global -> LDS loads: wave w fills the 8-row groups w, w+8, w+16, w+24 of both slices ----
    // Buffer loads: the resource starts at the tile's first row and this
    // slice's first k, and its size ends at row M (N), so rows past the end
    // read as zero.  The lane offsets are the same for A and W.
    const int lrow = lane >> 3;
    const int lchunk = (lane & 7) ^ lrow ^ (wave & 1);   // logical k chunk landing at this lane's LDS position
    uint32_t voff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) voff[i] = (uint32_t)(((wave + 8 * i) * 8 + lrow) * K + 8 * lchunk) * 2u;
    const int nkt = (MODE == kFp32 && splits > 1) ? K / splits / TK : K / TK;
    auto issue = [&](int kt, uint16_t* la, uint16_t* lw) __attribute__((always_inline)) {
        const int k0 = kt * TK;
        const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(A + (int64_t)m0 * K + k0), 0, (int)(((int64_t)(M - m0) * K - k0) * 2), 0x00020000);
        const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(W + (int64_t)n0 * K + k0), 0, (int)(((int64_t)(N - n0) * K - k0) * 2), 0x00020000);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, la + (wave + 8 * i) * 8 * TK, 16, (int)voff[i], 0, 0, 0);
            if (i < TN / 64)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, lw + (wave + 8 * i) * 8 * TK, 16, (int)voff[i], 0, 0, 0);
        }
    };

    f16v acc[2][RB];     // [column block][row block]; fp32 partials of the current K group
    h2_t H[2][RB][8];    // fp16 accumulators
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < RB; ++j)
#pragma unroll
            for (int p = 0; p < 8; ++p) H[i][j][p] = (h2_t){(_Float16)0.f, (_Float16)0.f};

    int ks = 0;   // 16-wide k steps done (group index of the partial dump)
    // end of a K group: fold the partials into H (or dump them); the next
    // group's first MFMA starts from a zero accumulator
    auto group_end = [&]() __attribute__((always_inline)) {
        if constexpr (MODE == kPartial) {
            const int g = (ks * 16 - 1) / gk;
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < RB; ++j) {
                    const int m = m0 + wm + 32 * j + (lane & 31);
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int n = n0 + wn + 32 * i + 8 * (r / 4) + 4 * (lane >> 5) + (r & 3);
                        if (m < M && n < N) P[((int64_t)g * M + m) * N + n] = acc[i][j][r];
                    }
                }
        } else if constexpr (MODE != kFp32) {
            fold_all<MODE, GN>(acc, H);
        }
    };

    // One 64-wide K slice from buffer BUF.  FRESH: the slice starts a K group;
    // FOLD: it ends one.  With group_k 16 / 32 (SMALLG) groups of GS steps
    // start and end inside the slice.
    auto stage = [&](int kt, auto buf_tag, auto fresh_tag, auto fold_tag) __attribute__((always_inline)) {
        constexpr int BUF = decltype(buf_tag)::value;
        constexpr bool FRESH = decltype(fresh_tag)::value;
        constexpr bool FOLD = decltype(fold_tag)::value;
        const uint16_t* la = BUF ? sA1 : sA0;
        const uint16_t* lw = BUF ? sW1 : sW0;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();                      // slice kt landed; the other buffer fully read
        if (kt + 1 < nkt) issue(kt + 1, BUF ? sA0 : sA1, BUF ? sW0 : sW1);
        // keep the prefetch ahead of this slice's compute: without the fence the
        // scheduler sinks the loads past it and the next wait exposes their latency
        __builtin_amdgcn_sched_barrier(0);
        // this lane's rows: wn + 32 i + lane % 32 of W, wm + 32 j + lane % 32 of A (row % 16 == lane % 16)
        const char* lwb = reinterpret_cast<const char*>(lw) + (wn + (lane & 31)) * (TK * 2);
        const char* lab = reinterpret_cast<const char*>(la) + (wm + (lane & 31)) * (TK * 2);
#pragma unroll
        for (int s = 0; s < TK / 16; ++s) {
            const int cs = swz_pos(lane & 15, 2 * s + (lane >> 5)) << 4;   // swizzled chunk, bytes
            h8 bop[2], aop[RB];
#pragma unroll
            for (int i = 0; i < 2; ++i) bop[i] = *reinterpret_cast<const h8*>(lwb + i * 32 * (TK * 2) + cs);
#pragma unroll
            for (int j = 0; j < RB; ++j) aop[j] = *reinterpret_cast<const h8*>(lab + j * 32 * (TK * 2) + cs);
            const bool zero = SMALLG ? (s % GS == 0) : (FRESH && s == 0);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < RB; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bop[i], aop[j], zero ? (f16v){} : acc[i][j],
                                                                       0, 0, 0);
            if constexpr (SMALLG) {
                if (s % GS == GS - 1) {
                    ks += GS;
                    group_end();
                }
            }
        }
        if constexpr (!SMALLG) {
            ks += TK / 16;
            if constexpr (FOLD) group_end();
        }
    };
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    using T_ = std::true_type;
    using F_ = std::false_type;

    issue(0, sA0, sW0);
    int kt = 0;
    if constexpr (MODE == kFp32) {   // one group over all of K
        stage(0, B0{}, T_{}, F_{});
        for (kt = 1; kt + 1 < nkt; kt += 2) {
            stage(kt, B1{}, F_{}, F_{});
            stage(kt + 1, B0{}, F_{}, F_{});
        }
        if (kt < nkt) stage(kt, B1{}, F_{}, F_{});
    } else if constexpr (SMALLG || SPG == 1) {
        for (; kt + 1 < nkt; kt += 2) {
            stage(kt, B0{}, T_{}, T_{});
            stage(kt + 1, B1{}, T_{}, T_{});
        }
        if (kt < nkt) stage(kt, B0{}, T_{}, T_{});
    } else if constexpr (SPG == 2) {
        for (; kt < nkt; kt += 2) {
            stage(kt, B0{}, T_{}, F_{});
            stage(kt + 1, B1{}, F_{}, T_{});
        }
    } else {
        for (; kt < nkt; kt += 4) {
            stage(kt, B0{}, T_{}, F_{});
            stage(kt + 1, B1{}, F_{}, F_{});
            stage(kt + 2, B0{}, F_{}, F_{});
            stage(kt + 3, B1{}, F_{}, T_{});
        }
    }

    if constexpr (MODE == kPartial) return;
    if constexpr (MODE == kFp32) {
        if (splits > 1) {   // this K range's fp32 sums, 4 columns a store
            float* Ps = P + (int64_t)split * M * N;
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < RB; ++j) {
                    const int m = m0 + wm + 32 * j + (lane & 31);
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int n = n0 + wn + 32 * i + 8 * q + 4 * (lane >> 5);
                        if (m < M && n < N)
                            *reinterpret_cast<float4*>(Ps + (int64_t)m * N + n) =
                                make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                                            acc[i][j][4 * q + 3]);
                    }
                }
            return;
        }
    }

    // ---- store: each wave stages its WROWS x 64 fp16 sub-tile in LDS, then writes full row segments ----
    static_assert(8 * WROWS * 64 <= 2 * SLICE + 2 * WSL, "staging area");
    __syncthreads();
    uint16_t* st = smem + wave * (WROWS * 64);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < RB; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                h2_t lo, hi;
                if constexpr (MODE == kFp32) {
                    lo = cvt2(acc[i][j][4 * q], acc[i][j][4 * q + 1]);
                    hi = cvt2(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
                } else {
                    lo = H[i][j][2 * q];
                    hi = H[i][j][2 * q + 1];
                }
                const int row = 32 * j + (lane & 31);
                *reinterpret_cast<uint2*>(st + swz(row, 4 * i + q) + 4 * (lane >> 5)) =
                    make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
            }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < WROWS / 8; ++t) {
        const int id = lane + 64 * t;
        const int row = id >> 3, ch = id & 7;
        const u32x4 v = *reinterpret_cast<const u32x4*>(st + swz(row, ch));
        const int m = m0 + wm + row, n = n0 + wn + 8 * ch;
        if (m < M && n < N) *reinterpret_cast<u32x4*>(C + (int64_t)m * ldc + n) = v;
    }
}

template <int MODE, int GN, int TN>
void launch(const void* A, const void* W, void* C, float* P, int M, int N, int K, int gk, hipStream_t st,
            int splits = 1, int batches = 1, int64_t sA = 0, int64_t sW = 0, int64_t sC = 0, int wgroup = 1,
            int64_t ldc = 0) {
    const int tm = (M + TM - 1) / TM, tn = (N + TN - 1) / TN;
    if (ldc == 0) ldc = N;
    const dim3 grid(tm * tn * (splits > batches ? splits : batches)), block(NT);
#define T256_LAUNCH(SM, GS_, SPG_)                                                                              \
    hipLaunchKernelGGL((kernel<MODE, GN, SM, GS_, SPG_, TN>), grid, block, 0, st, (const uint16_t*)A,          \
                       (const uint16_t*)W, (uint16_t*)C, P, M, N, K, gk, tm, tn, splits, batches, sA, sW, sC, wgroup,  \
                       ldc)
    if constexpr (MODE == kFp32) {
        T256_LAUNCH(false, 4, 1);
    } else {
        if (gk == 64) T256_LAUNCH(false, 4, 1);
        else if (gk == 128) T256_LAUNCH(false, 4, 2);
        else T256_LAUNCH(false, 4, 4);
    }
#undef T256_LAUNCH
}

}  // namespace t256

template <int TN>
static int launch_w(int mode, int gn, const void* A, const void* B, void* C, float* P, int M, int N, int K, int gk,
                    hipStream_t st) {
    using namespace t256;
    switch (mode) {
        case kGrouped: launch<kGrouped, 4, TN>(A, B, C, P, M, N, K, gk, st); return 1;
        case kFp32: launch<kFp32, 4, TN>(A, B, C, P, M, N, K, gk, st); return 1;
        case kPartial: launch<kPartial, 4, TN>(A, B, C, P, M, N, K, gk, st); return 1;
        case kInt8:
            switch (gn) {
                case 4: launch<kInt8, 4, TN>(A, B, C, P, M, N, K, gk, st); return 1;
                case 8: launch<kInt8, 8, TN>(A, B, C, P, M, N, K, gk, st); return 1;
                case 16: launch<kInt8, 16, TN>(A, B, C, P, M, N, K, gk, st); return 1;
                case 32: launch<kInt8, 32, TN>(A, B, C, P, M, N, K, gk, st); return 1;
            }
            return 0;
        case kFp8:
            switch (gn) {
                case 4: launch<kFp8, 4, TN>(A, B, C, P, M, N, K, gk, st); return 1;
                case 8: launch<kFp8, 8, TN>(A, B, C, P, M, N, K, gk, st); return 1;
                case 16: launch<kFp8, 16, TN>(A, B, C, P, M, N, K, gk, st); return 1;
                case 32: launch<kFp8, 32, TN>(A, B, C, P, M, N, K, gk, st); return 1;
            }
            return 0;
    }
    return 0;
}

namespace {

int cu_count() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess)
            cus = n;
    }
    return cus;
}

// C = R16(P[0] + P[1] + ...) in split order, 8 outputs a thread (M * N % 8 == 0)
__global__ __launch_bounds__(256) void splitk_sum_kernel(const float* __restrict__ P, uint16_t* __restrict__ C,
                                                         int64_t mn, int splits) {
    const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (u * 8 >= mn) return;
    float v[8];
    const float4* p0 = reinterpret_cast<const float4*>(P + 8 * u);
    const float4 a = p0[0], b = p0[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    for (int s = 1; s < splits; ++s) {
        const float4* ps = reinterpret_cast<const float4*>(P + (int64_t)s * mn + 8 * u);
        const float4 c = ps[0], d = ps[1];
        v[0] += c.x; v[1] += c.y; v[2] += c.z; v[3] += c.w; v[4] += d.x; v[5] += d.y; v[6] += d.z; v[7] += d.w;
    }
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) w[q] = __builtin_bit_cast(uint32_t, cvt2(v[2 * q], v[2 * q + 1]));
    *reinterpret_cast<uint4*>(C + 8 * u) = make_uint4(w[0], w[1], w[2], w[3]);
}

}  // namespace

int splitk_fp32_splits(int M, int N, int K) {
    using namespace t256;
    const int cus = cu_count();
    if (cus <= 0 || M < 1 || N % 8 != 0 || K % (2 * TK) != 0) return 1;
    if ((int64_t)M * K >= (1ll << 31) || (int64_t)N * K >= (1ll << 31)) return 1;
    const int64_t tm = (M + TM - 1) / TM;
    const int64_t t256 = tm * ((N + 255) / 256), t128 = tm * ((N + 127) / 128);
    // long K on a grid of at most one round of 256x128 tiles: two K halves on 256x256
    // tiles fill the same round with the more efficient tile (prefill down projection,
    // M = 2048, K = 14336, N = 4096: 201 + 13 us against 294 us); the fp32 partials cost
    // 2 x 2 x M x N x 4 bytes of traffic, which shorter K does not repay (o projection,
    // K = 4096: 74 + 13 us against 85 us)
    if (t128 <= cus && 2 * t256 <= cus && K >= 8192) return 2;
    return 1;
}

int launch_splitk_fp32(const void* A, const void* W, void* C, float* ws, int M, int N, int K, int splits,
                       hipStream_t st) {
    using namespace t256;
    if (splits < 2 || (K / splits) % TK != 0) return 0;
    if (((uintptr_t)A | (uintptr_t)W | (uintptr_t)C | (uintptr_t)ws) % 16 != 0) return 0;
    launch<kFp32, 4, 256>(A, W, nullptr, ws, M, N, K, K / splits, st, splits);
    const int64_t mn = (int64_t)M * N;
    hipLaunchKernelGGL(splitk_sum_kernel, dim3((unsigned)((mn / 8 + 255) / 256)), dim3(256), 0, st, ws,
                       (uint16_t*)C, mn, splits);
    return 1;
}

int launch_batched_fp32(const void* A, const void* W, void* C, int batches, int M, int N, int K, int64_t sA,
                        int64_t sW, int64_t sC, int wgroup, int64_t ldc, hipStream_t st) {
    using namespace t256;
    if (batches < 1 || M < 1 || N < 1 || K % TK != 0 || N % 8 != 0 || wgroup < 1 || ldc < N) return 0;
    if (((uintptr_t)A | (uintptr_t)W | (uintptr_t)C) % 16 != 0 || (sA | sW | sC | ldc) % 8 != 0) return 0;
    if ((int64_t)M * K >= (1ll << 31) || (int64_t)N * K >= (1ll << 31)) return 0;
    if (sA < (int64_t)M * K || sW < (int64_t)N * K) return 0;
    const int64_t tiles = (int64_t)batches * ((M + TM - 1) / TM) * ((N + 255) / 256);
    if (tiles * 2 > 0x7fffffffll) return 0;
    if (N <= 128) launch<kFp32, 4, 128>(A, W, C, nullptr, M, N, K, K, st, 1, batches, sA, sW, sC, wgroup, ldc);
    else launch<kFp32, 4, 256>(A, W, C, nullptr, M, N, K, K, st, 1, batches, sA, sW, sC, wgroup, ldc);
    return 1;
}

int launch_tile256(int mode, int gn, const void* A, const void* B, void* C, float* P, int M, int N, int K, int gk,
                   int b_is_nk, hipStream_t st) {
    using namespace t256;
    if (!b_is_nk || K % TK != 0 || N % 8 != 0 || M < 1 || N < 1) return 0;
    // group_k 16 / 32 (grouped accumulation, group partials) stay on the 128x128 kernel
    if (mode != kFp32 && (K % gk != 0 || (gk != 64 && gk != 128 && gk != 256))) return 0;
    if (((uintptr_t)A | (uintptr_t)B | (uintptr_t)C) % 16 != 0) return 0;
    // 32-bit element offsets inside the kernel
    if ((int64_t)M * K >= (1ll << 31) || (int64_t)N * K >= (1ll << 31)) return 0;
    if (mode == kFp32) gk = K;
    // fewer 256x256 tiles than compute units would leave most of the chip idle: the
    // 128x128 kernel fills it better
    const int cus = cu_count();
    const int64_t tm = (M + TM - 1) / TM;
    // psum-quantized modes: 256x128 tiles when 256x256 tiles leave a partly empty last
    // round that 256x128 tiles fill (configs[2] gate/up: 896 tiles = 3.5 rounds against
    // 1792 = 7; 3% faster).  With whole rounds either way the 256x256 tiles are faster
    // (configs[3]: 0.39 against 0.45 ms), as they are for fp32 / grouped accumulation.
    if (mode == kInt8 || mode == kFp8) {
        const int64_t t256 = tm * ((N + 255) / 256), t128 = tm * ((N + 127) / 128);
        const double e256 = (double)t256 / (double)(((t256 + cus - 1) / cus) * cus);
        const double e128 = (double)t128 / (double)(((t128 + cus - 1) / cus) * cus);
        if (t128 >= 2 * cus && e128 > e256 + 0.05) return launch_w<128>(mode, gn, A, B, C, P, M, N, K, gk, st);
    }
    const int64_t t256 = tm * ((N + 255) / 256), t128 = tm * ((N + 127) / 128);
    if (t256 >= cus) return launch_w<256>(mode, gn, A, B, C, P, M, N, K, gk, st);
    // fewer 256-wide tiles than compute units: one round of them costs about 1.3 rounds of
    // 128-wide tiles, so they win whenever the 128-wide tiles need two rounds or more
    // (prefill q/k/v, M = 2048, N = 6144: 192 tiles in 105 us against 384 in 149 us)
    if (t128 > cus) return launch_w<256>(mode, gn, A, B, C, P, M, N, K, gk, st);
    if (t128 == cus) return launch_w<128>(mode, gn, A, B, C, P, M, N, K, gk, st);
    return 0;
}

}  // namespace hbq_gemm
