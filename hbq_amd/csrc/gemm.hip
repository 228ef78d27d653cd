// Block-quant GEMMs of blockquant_ext on gfx950 MFMA: the C-ABI entry points,
// the 128x128-tile kernel and the pure-fp16 FMA-chain kernel.
//
// C[M,N] (fp16) = A[M,K] (fp16) x B[K,N] (fp16), with B either row-major
// [K,N] as the reference op takes it, or stored transposed as W[N,K] (the
// nn.Linear weight layout, which skips the caller's transpose copy).
//
// The K dimension is cut into groups of group_k.  Inside a group the fp32
// partial comes from v_mfma_f32_32x32x16_f16; at the end of each group the
// epilogue of gemm_common.h folds it into the fp16 accumulators as the
// reference does after its sequential fmaf chain; fp32 accumulation is one
// group spanning K, and the partial mode writes every group's fp32 partial.
//
// W[N,K] operands with K % 64 == 0 and group_k >= 64 go to the 256x256-tile
// kernel (gemm_tile256.hip); everything else runs here: 128x128 tiles, 4
// waves of 64x64, register-staged LDS double buffering, B[K,N] transposed into
// LDS by 16-bit scatters.  Both kernels issue the same MFMA sequence per
// output element, so they give the same bits.
#include <hip/hip_runtime.h>
#include <math.h>
#include <mutex>
#include <stdint.h>

#include "gemm_common.h"
#include "gemm_tile256.h"
#include "hbq_capi_internal.h"
#include "hbq_amd.h"

namespace hbq_gemm {

constexpr int BM = 128;          // output rows per workgroup
constexpr int BN = 128;          // output columns per workgroup
constexpr int BK = 64;           // K per LDS stage
constexpr int LDK = BK + 8;      // padded LDS row (halfs): 144 B, conflict-free 16 B reads
constexpr int kThreads = 256;

// ---- global -> LDS tile loads ----------------------------------------------
// A tile: rows m0..m0+BM, k0..k0+BK, k contiguous.  Chunk c (8 halfs): row c / 8, col (c % 8) * 8.
__device__ __forceinline__ u32x4 load_chunk(const uint16_t* __restrict__ base, int64_t ld, int64_t row, int64_t col,
                                            int64_t nrows, int64_t ncols, bool vec_ok) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (row >= nrows || col >= ncols) return v;
    const uint16_t* p = base + row * ld + col;
    if (vec_ok && col + 8 <= ncols) return *reinterpret_cast<const u32x4*>(p);
    uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; ++i)
        if (col + i < ncols) w[i / 2] |= (uint32_t)p[i] << (16 * (i % 2));
    v = (u32x4){w[0], w[1], w[2], w[3]};
    return v;
}

// ---- the kernel ------------------------------------------------------------
// SMALLG: group_k < BK (16 or 32), so group ends fall inside an LDS stage.
template <int MODE, int GN, bool BT, bool SMALLG>
__global__ __launch_bounds__(kThreads, 2) void gemm_kernel(const uint16_t* __restrict__ A,
                                                            const uint16_t* __restrict__ B,
                                                            uint16_t* __restrict__ C, float* __restrict__ P, int M,
                                                            int N, int K, int gk, int vec_a, int vec_b) {
    __shared__ __attribute__((aligned(16))) uint16_t As[2][BM][LDK];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN][LDK];   // stored transposed: [n][k]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = (wave & 1) * 64;     // wave's row offset in the tile
    const int wn = (wave >> 1) * 64;    // wave's column offset in the tile
    const int64_t m0 = (int64_t)blockIdx.y * BM;
    const int64_t n0 = (int64_t)blockIdx.x * BN;
    const int nkt = (K + BK - 1) / BK;

    f16v acc[2][2];     // [n block][m block]
    h2_t H[2][2][8];    // fp16 accumulators, packed pairs of adjacent columns
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            acc[i][j] = (f16v){};
#pragma unroll
            for (int p = 0; p < 8; ++p) H[i][j][p] = (h2_t){(_Float16)0.f, (_Float16)0.f};
        }

    // global tile loaders into registers
    u32x4 ra[4], rb[4];
    auto gload = [&](int kt) {
        const int64_t k0 = (int64_t)kt * BK;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int c = tid + i * kThreads;                    // 0..1023
            ra[i] = load_chunk(A, K, m0 + c / 8, k0 + (c % 8) * 8, M, K, vec_a);
        }
        if constexpr (BT) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                int c = tid + i * kThreads;
                rb[i] = load_chunk(B, K, n0 + c / 8, k0 + (c % 8) * 8, N, K, vec_b);
            }
        } else {
            // B[K,N]: chunk c covers k = c / 16, n = (c % 16) * 8 .. +7
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                int c = tid + i * kThreads;
                rb[i] = load_chunk(B, N, k0 + c / 16, n0 + (c % 16) * 8, K, N, vec_b);
            }
        }
    };
    auto swrite = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int c = tid + i * kThreads;
            *reinterpret_cast<u32x4*>(&As[buf][c / 8][(c % 8) * 8]) = ra[i];
        }
        if constexpr (BT) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                int c = tid + i * kThreads;
                *reinterpret_cast<u32x4*>(&Bs[buf][c / 8][(c % 8) * 8]) = rb[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                int c = tid + i * kThreads;
                int kk = c / 16, nn = (c % 16) * 8;
                uint32_t w[4] = {rb[i].x, rb[i].y, rb[i].z, rb[i].w};
#pragma unroll
                for (int e = 0; e < 8; ++e) Bs[buf][nn + e][kk] = (uint16_t)(w[e / 2] >> (16 * (e % 2)));
            }
        }
    };

    gload(0);
    swrite(0);
    __syncthreads();

    int ks_global = 0;   // k steps (16 wide) done
    const int nks = (K + 15) / 16;
    const int gsteps = gk / 16;
    // fold (or dump) the group partials and restart them
    auto group_end = [&]() {
        if constexpr (MODE == kPartial) {
            const int g = (ks_global * 16 - 1) / gk;
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int64_t m = m0 + wm + j * 32 + (lane & 31);
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int64_t n = n0 + wn + i * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r & 3);
                        if (m < M && n < N) P[((int64_t)g * M + m) * N + n] = acc[i][j][r];
                    }
                }
        } else {
            fold_all<MODE, GN>(acc, H);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] = (f16v){};
    };
    for (int kt = 0; kt < nkt; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nkt) gload(kt + 1);
#pragma unroll
        for (int s = 0; s < BK / 16; ++s) {
            if (ks_global >= nks) break;
            const int kk = s * 16 + 8 * (lane >> 5);
            h8 bop[2], aop[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                bop[i] = *reinterpret_cast<const h8*>(&Bs[buf][wn + i * 32 + (lane & 31)][kk]);
                aop[i] = *reinterpret_cast<const h8*>(&As[buf][wm + i * 32 + (lane & 31)][kk]);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bop[i], aop[j], acc[i][j], 0, 0, 0);
            ++ks_global;
            if constexpr (SMALLG && MODE != kFp32)
                if (ks_global % gsteps == 0 || ks_global == nks) group_end();
        }
        // group_k >= BK: groups end on stage boundaries (or at the ragged end of K)
        if constexpr (!SMALLG && MODE != kFp32)
            if (ks_global % gsteps == 0 || ks_global == nks) group_end();
        if (kt + 1 < nkt) swrite(buf ^ 1);
        __syncthreads();
    }

    if constexpr (MODE == kPartial) return;
    // write C: lane owns row m, columns in runs of 4
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int64_t m = m0 + wm + j * 32 + (lane & 31);
            if (m >= M) continue;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t n = n0 + wn + i * 32 + 8 * q + 4 * (lane >> 5);
                h2_t lo, hi;
                if constexpr (MODE == kFp32) {
                    lo = cvt2(acc[i][j][4 * q], acc[i][j][4 * q + 1]);
                    hi = cvt2(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
                } else {
                    lo = H[i][j][2 * q];
                    hi = H[i][j][2 * q + 1];
                }
                const uint32_t w0 = __builtin_bit_cast(uint32_t, lo), w1 = __builtin_bit_cast(uint32_t, hi);
                const uint16_t h[4] = {(uint16_t)w0, (uint16_t)(w0 >> 16), (uint16_t)w1, (uint16_t)(w1 >> 16)};
                uint16_t* dst = C + m * (int64_t)N + n;
                if (n + 4 <= N && ((((uintptr_t)dst) & 7) == 0)) {
                    *reinterpret_cast<uint2*>(dst) = make_uint2(w0, w1);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (n + e < N) dst[e] = h[e];
                }
            }
        }
}

// ---- pure fp16 accumulation (gemm.cu:96-303, FP16_ACCUM=true) ---------------
// acc = fma16(a, b, acc) over ascending k, one rounding per step: a VALU chain,
// since MFMA accumulates in fp32.  Each thread owns a 4x4 output tile.
constexpr int HT = 64, HK = 32;
__global__ __launch_bounds__(256) void gemm_fp16acc_kernel(const uint16_t* __restrict__ A,
                                                          const uint16_t* __restrict__ B, uint16_t* __restrict__ C,
                                                          int M, int N, int K, int bt) {
    __shared__ _Float16 sA[HK][HT + 2];
    __shared__ _Float16 sB[HK][HT + 2];
    const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
    const int64_t m0 = (int64_t)blockIdx.y * HT, n0 = (int64_t)blockIdx.x * HT;
    _Float16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = (_Float16)0.f;
    for (int k0 = 0; k0 < K; k0 += HK) {
        for (int e = threadIdx.x; e < HT * HK; e += 256) {
            int r = e / HK, c = e % HK;
            int64_t m = m0 + r, k = k0 + c;
            uint16_t va = (m < M && k < K) ? A[m * K + k] : 0;
            sA[c][r] = __builtin_bit_cast(_Float16, va);
            int64_t n = n0 + r;
            uint16_t vb = 0;
            if (n < N && k < K) vb = bt ? B[n * K + k] : B[k * (int64_t)N + n];
            sB[c][r] = __builtin_bit_cast(_Float16, vb);
        }
        __syncthreads();
        const int kend = (K - k0) < HK ? (K - k0) : HK;
        for (int k = 0; k < kend; ++k) {
            _Float16 a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) { a[i] = sA[k][ty * 4 + i]; b[i] = sB[k][tx * 4 + i]; }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf16(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int64_t m = m0 + ty * 4 + i, n = n0 + tx * 4 + j;
            if (m < M && n < N) C[m * N + n] = __builtin_bit_cast(uint16_t, acc[i][j]);
        }
}

// ---- 16-bit transpose (B[K,N] -> W[N,K] for the 256x256 kernel) ----------
// 64x64 tiles through LDS: 16-byte loads along the source rows, 16-byte stores
// along the destination rows.
constexpr int TT = 64;
__global__ __launch_bounds__(256) void transpose16_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                                                          int64_t rows, int64_t cols) {
    __shared__ uint16_t t[TT][TT + 2];
    const int64_t r0 = (int64_t)blockIdx.y * TT, c0 = (int64_t)blockIdx.x * TT;
    const bool vec = (cols % 8 == 0) && (rows % 8 == 0) && (((uintptr_t)src | (uintptr_t)dst) % 16 == 0);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int id = threadIdx.x + 256 * k;          // 512 chunks of 8 halfs
        const int rr = id / 8, cc = (id % 8) * 8;
        const int64_t r = r0 + rr, c = c0 + cc;
        uint16_t v[8];
        if (vec && r < rows && c + 8 <= cols) {
            const u32x4 q = *reinterpret_cast<const u32x4*>(src + r * cols + c);
            const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = (uint16_t)(w[e / 2] >> (16 * (e % 2)));
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = (r < rows && c + e < cols) ? src[r * cols + c + e] : (uint16_t)0;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) t[rr][cc + e] = v[e];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int id = threadIdx.x + 256 * k;
        const int cr = id / 8, rc = (id % 8) * 8;       // destination row (source column), 8 source rows
        const int64_t dr = c0 + cr, dc = r0 + rc;
        uint16_t v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = t[rc + e][cr];
        if (dr >= cols) continue;
        if (vec && dc + 8 <= rows) {
            *reinterpret_cast<u32x4*>(dst + dr * rows + dc) =
                (u32x4){(uint32_t)v[0] | ((uint32_t)v[1] << 16), (uint32_t)v[2] | ((uint32_t)v[3] << 16),
                        (uint32_t)v[4] | ((uint32_t)v[5] << 16), (uint32_t)v[6] | ((uint32_t)v[7] << 16)};
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (dc + e < rows) dst[dr * rows + dc + e] = v[e];
        }
    }
}

}  // namespace hbq_gemm

using namespace hbq_gemm;

namespace {

template <int MODE, int GN, bool BT, bool SMALLG>
void launch(const void* A, const void* B, void* C, float* P, int M, int N, int K, int gk, hipStream_t st) {
    dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
    int vec_a = (K % 8 == 0) && (((uintptr_t)A) % 16 == 0);
    int vec_b = (BT ? (K % 8 == 0) : (N % 8 == 0)) && (((uintptr_t)B) % 16 == 0);
    hipLaunchKernelGGL((gemm_kernel<MODE, GN, BT, SMALLG>), grid, dim3(kThreads), 0, st, (const uint16_t*)A,
                       (const uint16_t*)B, (uint16_t*)C, P, M, N, K, gk, vec_a, vec_b);
}

// the 128x128 kernel for every case the 256x256 one does not take
template <int MODE, int GN>
void launch_any(const void* A, const void* B, void* C, float* P, int M, int N, int K, int gk, int b_is_nk,
                hipStream_t st) {
    if (launch_tile256(MODE, GN, A, B, C, P, M, N, K, gk, b_is_nk, st)) return;
    const bool small = gk < BK;
    if (b_is_nk) {
        if (small) launch<MODE, GN, true, true>(A, B, C, P, M, N, K, gk, st);
        else launch<MODE, GN, true, false>(A, B, C, P, M, N, K, gk, st);
    } else {
        if (small) launch<MODE, GN, false, true>(A, B, C, P, M, N, K, gk, st);
        else launch<MODE, GN, false, false>(A, B, C, P, M, N, K, gk, st);
    }
}

template <int MODE>
int psum_dispatch(int gk, int gn, const void* A, const void* B, void* C, int M, int N, int K, int b_is_nk,
                  hipStream_t st) {
    switch (gn) {
        case 4: launch_any<MODE, 4>(A, B, C, nullptr, M, N, K, gk, b_is_nk, st); return 0;
        case 8: launch_any<MODE, 8>(A, B, C, nullptr, M, N, K, gk, b_is_nk, st); return 0;
        case 16: launch_any<MODE, 16>(A, B, C, nullptr, M, N, K, gk, b_is_nk, st); return 0;
        case 32: launch_any<MODE, 32>(A, B, C, nullptr, M, N, K, gk, b_is_nk, st); return 0;
    }
    return hbq_fail(HBQ_ERR_INVALID, "group_n must be one of {4,8,16,32}");
}

int check_shapes(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K) {
    if (M < 0 || N < 0 || K < 0) return hbq_fail(HBQ_ERR_INVALID, "negative GEMM shape");
    if ((A == nullptr && M * K > 0) || (B == nullptr && K * N > 0) || (C == nullptr && M * N > 0))
        return hbq_fail(HBQ_ERR_INVALID, "null tensor pointer");
    if (M > 0x7fffffff / 1 || N > 0x7fffffff || K > 0x7fffffff) return hbq_fail(HBQ_ERR_INVALID, "GEMM too large");
    if ((M + BM - 1) / BM > 65535) return hbq_fail(HBQ_ERR_INVALID, "M too large for one launch");
    return 0;
}

__global__ void zero_fill_kernel(uint16_t* __restrict__ C, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) C[i] = 0;
}

// K == 0: every output is +0 (an empty sum folded into a +0 accumulator).  A
// fill kernel rather than hipMemsetAsync, so the call stays graph-capturable.
int zero_output(void* C, int64_t M, int64_t N, hipStream_t st) {
    int64_t n = M * N;
    if (n == 0) return 0;
    hipLaunchKernelGGL(zero_fill_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, (uint16_t*)C, n);
    return 0;
}

// ---------------------------------------------------------------------------
// Scratch of the allocation-free entry point (hbq_gemm_fp32_accum_noalloc): the
// split-K fp32 partials in a file-scope device array, one copy on every GPU the
// library runs on, held until the process ends.  Its name is a host-side stand-in
// for the symbol, not a device address: host code takes each device's address from
// hipGetSymbolAddress (first call on that device, with it current) and passes that.
// The split kernel writes every partial of the shape before the sum reads it, so
// nothing needs clearing between calls; calls that overlap on one GPU race on it.
// ---------------------------------------------------------------------------
constexpr int64_t kNoAllocScratchBytes = HBQ_NOALLOC_SCRATCH_BYTES;   // 2 splits x 2048 x 4096 fp32
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kScratchDevices];

int scratch_ptr(float** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hbq_fail(HBQ_ERR_HIP, "hipGetDevice failed: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kScratchDevices) return hbq_fail(HBQ_ERR_UNSUPPORTED, "device index %d out of range", dev);
    std::lock_guard<std::mutex> g(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr)
            return hbq_fail(HBQ_ERR_HIP, "hipGetSymbolAddress of the scratch buffer failed: %s", hipGetErrorString(e));
        g_scratch_ptr[dev] = (float*)p;
    }
    *out = g_scratch_ptr[dev];
    return 0;
}

}  // namespace

extern "C" {

int hbq_gemm_fp32_accum_noalloc(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
                                int b_is_nk, void* stream) {
    hbq_clear_error();
    if (int rc = check_shapes(A, B, C, M, N, K)) return rc;
    hipStream_t st = (hipStream_t)stream;
    if (M == 0 || N == 0) return 0;
    if (K == 0) return zero_output(C, M, N, st);
    const int64_t need = hbq_gemm_fp32_accum_workspace(M, N, K, b_is_nk);
    if (need > kNoAllocScratchBytes)
        return hbq_fail(HBQ_ERR_INVALID,
                        "gemm_fp32_accum_noalloc: the split-K partials of this shape take %lld bytes, more than the "
                        "%lld-byte scratch buffer (use hbq_gemm_fp32_accum_ws with a workspace)",
                        (long long)need, (long long)kNoAllocScratchBytes);
    if (need > 0) {
        float* ws = nullptr;
        if (int rc = scratch_ptr(&ws)) return rc;
        if (launch_splitk_fp32(A, B, C, ws, (int)M, (int)N, (int)K,
                               (int)(need / ((int64_t)sizeof(float) * M * N)), st))
            return hbq_check_launch("gemm_fp32_accum_noalloc (split K)");
    }
    launch_any<kFp32, 4>(A, B, C, nullptr, (int)M, (int)N, (int)K, (int)K, b_is_nk, st);
    return hbq_check_launch("gemm_fp32_accum_noalloc");
}

int hbq_gemm_fp32_accum(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, int b_is_nk,
                        void* stream) {
    hbq_clear_error();
    if (int rc = check_shapes(A, B, C, M, N, K)) return rc;
    hipStream_t st = (hipStream_t)stream;
    if (M == 0 || N == 0) return 0;
    if (K == 0) return zero_output(C, M, N, st);
    launch_any<kFp32, 4>(A, B, C, nullptr, (int)M, (int)N, (int)K, (int)K, b_is_nk, st);
    return hbq_check_launch("gemm_fp32_accum");
}

int64_t hbq_gemm_fp32_accum_workspace(int64_t M, int64_t N, int64_t K, int b_is_nk) {
    if (!b_is_nk || M < 1 || N < 1 || K < 1 || M > 0x7fffffff || N > 0x7fffffff || K > 0x7fffffff) return 0;
    const int s = splitk_fp32_splits((int)M, (int)N, (int)K);
    return s > 1 ? (int64_t)s * M * N * (int64_t)sizeof(float) : 0;
}

int hbq_gemm_fp32_accum_ws(const void* A, const void* B, void* C, void* ws, int64_t ws_bytes, int64_t M, int64_t N,
                           int64_t K, int b_is_nk, void* stream) {
    hbq_clear_error();
    if (int rc = check_shapes(A, B, C, M, N, K)) return rc;
    if (ws_bytes < 0) return hbq_fail(HBQ_ERR_INVALID, "negative workspace size");
    hipStream_t st = (hipStream_t)stream;
    if (M == 0 || N == 0) return 0;
    if (K == 0) return zero_output(C, M, N, st);
    const int64_t need = hbq_gemm_fp32_accum_workspace(M, N, K, b_is_nk);
    if (need > 0 && ws != nullptr && ws_bytes >= need &&
        launch_splitk_fp32(A, B, C, (float*)ws, (int)M, (int)N, (int)K, (int)(need / ((int64_t)sizeof(float) * M * N)),
                           st))
        return hbq_check_launch("gemm_fp32_accum (split K)");
    launch_any<kFp32, 4>(A, B, C, nullptr, (int)M, (int)N, (int)K, (int)K, b_is_nk, st);
    return hbq_check_launch("gemm_fp32_accum");
}

int hbq_gemm_fp32_accum_batched_ex(const void* A, const void* W, void* C, int64_t batches, int64_t M, int64_t N,
                                   int64_t K, int64_t stride_a, int64_t stride_w, int64_t w_group, int64_t stride_c,
                                   int64_t ldc, void* stream) {
    hbq_clear_error();
    if (batches < 0) return hbq_fail(HBQ_ERR_INVALID, "negative batch count");
    if (int rc = check_shapes(A, W, C, M, N, K)) return rc;
    if (batches > 0x7fffffff) return hbq_fail(HBQ_ERR_INVALID, "too many batches");
    if (w_group < 1 || w_group > 0x7fffffff) return hbq_fail(HBQ_ERR_INVALID, "w_group must be at least 1");
    if (ldc < N) return hbq_fail(HBQ_ERR_INVALID, "ldc smaller than N");
    if (stride_a < M * K || stride_w < N * K) return hbq_fail(HBQ_ERR_INVALID, "batch strides smaller than one problem");
    // the problems' outputs must not overlap: one after another, or interleaved within the rows
    const bool apart = M == 0 || stride_c >= (M - 1) * ldc + N;
    const bool interleaved = stride_c >= N && (batches - 1) * stride_c + N <= ldc;
    if (batches > 1 && !apart && !interleaved) return hbq_fail(HBQ_ERR_INVALID, "the problems' outputs overlap");
    hipStream_t st = (hipStream_t)stream;
    if (batches == 0 || M == 0 || N == 0) return 0;
    if (K == 0) {
        if (ldc != N) return hbq_fail(HBQ_ERR_UNSUPPORTED, "K == 0 with ldc != N");
        for (int64_t z = 0; z < batches; ++z) zero_output((uint16_t*)C + z * stride_c, M, N, st);
        return hbq_check_launch("gemm_fp32_accum_batched");
    }
    if (!launch_batched_fp32(A, W, C, (int)batches, (int)M, (int)N, (int)K, stride_a, stride_w, stride_c, (int)w_group,
                             ldc, st)) {
        if (ldc != N)
            return hbq_fail(HBQ_ERR_UNSUPPORTED, "ldc != N needs K %% 64 == 0, N %% 8 == 0 and 16-byte aligned rows");
        for (int64_t z = 0; z < batches; ++z)
            launch_any<kFp32, 4>((const uint16_t*)A + z * stride_a, (const uint16_t*)W + (z / w_group) * stride_w,
                                 (uint16_t*)C + z * stride_c, nullptr, (int)M, (int)N, (int)K, (int)K, 1, st);
    }
    return hbq_check_launch("gemm_fp32_accum_batched");
}

int hbq_gemm_fp32_accum_batched(const void* A, const void* W, void* C, int64_t batches, int64_t M, int64_t N,
                                int64_t K, int64_t stride_a, int64_t stride_w, int64_t stride_c, void* stream) {
    if (stride_c < M * N) {
        hbq_clear_error();
        return hbq_fail(HBQ_ERR_INVALID, "batch strides smaller than one problem");
    }
    return hbq_gemm_fp32_accum_batched_ex(A, W, C, batches, M, N, K, stride_a, stride_w, 1, stride_c, N, stream);
}

int hbq_gemm_fp16_accum(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, int b_is_nk,
                        void* stream) {
    hbq_clear_error();
    if (int rc = check_shapes(A, B, C, M, N, K)) return rc;
    hipStream_t st = (hipStream_t)stream;
    if (M == 0 || N == 0) return 0;
    if (K == 0) return zero_output(C, M, N, st);
    dim3 grid((unsigned)((N + HT - 1) / HT), (unsigned)((M + HT - 1) / HT));
    hipLaunchKernelGGL(gemm_fp16acc_kernel, grid, dim3(256), 0, st, (const uint16_t*)A, (const uint16_t*)B,
                       (uint16_t*)C, (int)M, (int)N, (int)K, b_is_nk);
    return hbq_check_launch("gemm_fp16_accum");
}

int hbq_gemm_fp16_grouped_accum(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, int group_k,
                                int b_is_nk, void* stream) {
    hbq_clear_error();
    if (group_k != 16 && group_k != 32 && group_k != 64 && group_k != 128)
        return hbq_fail(HBQ_ERR_INVALID, "group_k must be one of {16,32,64,128}");
    if (int rc = check_shapes(A, B, C, M, N, K)) return rc;
    hipStream_t st = (hipStream_t)stream;
    if (M == 0 || N == 0) return 0;
    if (K == 0) return zero_output(C, M, N, st);
    launch_any<kGrouped, 4>(A, B, C, nullptr, (int)M, (int)N, (int)K, group_k, b_is_nk, st);
    return hbq_check_launch("gemm_fp16_grouped_accum");
}

static int psum_common(int mode, const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, int gk,
                       int gn, int b_is_nk, void* stream, const char* name) {
    hbq_clear_error();
    if (gk != 64 && gk != 128 && gk != 256) return hbq_fail(HBQ_ERR_INVALID, "group_k must be one of {64,128,256}");
    if (gn != 4 && gn != 8 && gn != 16 && gn != 32) return hbq_fail(HBQ_ERR_INVALID, "group_n must be one of {4,8,16,32}");
    if (int rc = check_shapes(A, B, C, M, N, K)) return rc;
    if (K % gk) return hbq_fail(HBQ_ERR_INVALID, "K must be divisible by group_k");
    if (N % gn) return hbq_fail(HBQ_ERR_INVALID, "N must be divisible by group_n");
    hipStream_t st = (hipStream_t)stream;
    if (M == 0 || N == 0) return 0;
    if (K == 0) return zero_output(C, M, N, st);
    const int rc = mode == kInt8 ? psum_dispatch<kInt8>(gk, gn, A, B, C, (int)M, (int)N, (int)K, b_is_nk, st)
                                 : psum_dispatch<kFp8>(gk, gn, A, B, C, (int)M, (int)N, (int)K, b_is_nk, st);
    if (rc) return rc;
    return hbq_check_launch(name);
}

int hbq_gemm_blockquant_mxint8(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, int group_k,
                               int group_n, int b_is_nk, void* stream) {
    return psum_common(kInt8, A, B, C, M, N, K, group_k, group_n, b_is_nk, stream, "gemm_blockquant_mxint8");
}

int hbq_gemm_blockquant_mxfp8(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, int group_k,
                              int group_n, int b_is_nk, void* stream) {
    return psum_common(kFp8, A, B, C, M, N, K, group_k, group_n, b_is_nk, stream, "gemm_blockquant_mxfp8");
}

int hbq_transpose16(const void* src, void* dst, int64_t rows, int64_t cols, void* stream) {
    hbq_clear_error();
    if (rows < 0 || cols < 0) return hbq_fail(HBQ_ERR_INVALID, "negative shape");
    if (rows == 0 || cols == 0) return 0;
    if (src == nullptr || dst == nullptr) return hbq_fail(HBQ_ERR_INVALID, "null tensor pointer");
    const int64_t gx = (cols + TT - 1) / TT, gy = (rows + TT - 1) / TT;
    if (gx > 0x7fffffff || gy > 65535) return hbq_fail(HBQ_ERR_INVALID, "tensor too large for one launch");
    hipLaunchKernelGGL(transpose16_kernel, dim3((unsigned)gx, (unsigned)gy), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)src, (uint16_t*)dst, rows, cols);
    return hbq_check_launch("transpose16");
}

int hbq_gemm_group_partials(const void* A, const void* B, void* P, int64_t M, int64_t N, int64_t K, int group_k,
                            int b_is_nk, void* stream) {
    hbq_clear_error();
    // the ops' group sizes, or any multiple of the 128x128 kernel's K stage (a split-K half)
    if (group_k != 16 && group_k != 32 && (group_k < 64 || group_k % BK != 0))
        return hbq_fail(HBQ_ERR_INVALID, "group_k must be 16, 32 or a multiple of %d", BK);
    if (int rc = check_shapes(A, B, P, M, N, K)) return rc;
    if (M == 0 || N == 0 || K == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    launch_any<kPartial, 4>(A, B, nullptr, (float*)P, (int)M, (int)N, (int)K, group_k, b_is_nk, st);
    return hbq_check_launch("gemm_group_partials");
}

}  // extern "C"
