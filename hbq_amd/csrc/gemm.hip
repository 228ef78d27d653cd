// Block-quant GEMMs of blockquant_ext on gfx950 MFMA.
//
// C[M,N] (fp16) = A[M,K] (fp16) x B[K,N] (fp16), with B either row-major
// [K,N] as the reference op takes it, or stored transposed as W[N,K] (the
// nn.Linear weight layout, which skips the caller's transpose copy).
//
// The K dimension is cut into groups of GK.  Inside a group the fp32 partial
// comes from v_mfma_f32_32x32x16_f16; at the end of each group an epilogue
// fused into the kernel folds the partial into an fp16 accumulator exactly as
// the reference does after its sequential fmaf chain
// (blockquant_ext_src/gemm.cu:354-377, 810-887, 1198-1277):
//   grouped : H = R16(H + R16(P))
//   mxint8  : per (row, GN columns) s = 2^(ilogb(max|P|) - 6), Q = clamp(rne(P/s), +-127) * s,
//             H = R16(H + R16(Q))
//   mxfp8   : same with E3M4 quantize-dequantize and s = 2^(ilogb(max|P|) - 3)
//   fp32    : one group spanning K, C = R16(P)
//   partial : P of every group written out (fp32), for checking the epilogue
//
// Operand order is swapped (D = B^T A^T): the MFMA "row" is the output column
// n and the MFMA "column" is the output row m, so lane l owns row m = l % 32
// of a 32x32 block and 16 of its 32 columns (n = 8*(r/4) + 4*(l/32) + r%4);
// the other 16 sit in lane l ^ 32.  A psum group of up to 32 columns of one
// row therefore needs one cross-lane exchange.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "hbq_capi_internal.h"

namespace hbq_gemm {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

enum Mode : int { kGrouped = 0, kInt8 = 1, kFp8 = 2, kFp32 = 3, kPartial = 4 };

constexpr int BM = 128;          // output rows per workgroup
constexpr int BN = 128;          // output columns per workgroup
constexpr int BK = 64;           // K per LDS stage
constexpr int LDK = BK + 8;      // padded LDS row (halfs): 144 B, conflict-free 16 B reads
constexpr int kThreads = 256;

__device__ __forceinline__ float f16r(float v) {
    _Float16 h = (_Float16)v;
    asm("" : "+v"(h));
    return (float)h;
}

// ---- psum quantizers (gemm.cu:677-745, 1145-1251) --------------------------
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

// Fold the 16 fp32 partials of one 32x32 block into the fp16 accumulators.
template <int MODE, int GN>
__device__ __forceinline__ void fold_block(f16v& acc, float* H) {
    if constexpr (MODE == kGrouped) {
#pragma unroll
        for (int r = 0; r < 16; ++r) H[r] = f16r(H[r] + f16r(acc[r]));
    } else {
        // registers of one column group: GN=4 -> r/4 within a lane-half pair, else r/(GN/2) across l^32
        constexpr int RPG = GN >= 8 ? GN / 2 : 4;     // registers per group in this lane
        constexpr int NG = 16 / RPG;
        constexpr int shift = MODE == kInt8 ? 6 : 3;
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            float mx = 0.f;
#pragma unroll
            for (int r = g * RPG; r < (g + 1) * RPG; ++r) mx = fmaxf(mx, fabsf(acc[r]));
            if constexpr (GN >= 8) mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float s = psum_scale(mx, shift);
            const float inv = 1.f / s;
#pragma unroll
            for (int r = g * RPG; r < (g + 1) * RPG; ++r) {
                float q = MODE == kInt8 ? int8_qdq(acc[r], s, inv) : e3m4_qdq(acc[r], s);
                H[r] = f16r(H[r] + f16r(q));
            }
        }
    }
}

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
template <int MODE, int GK, int GN, bool BT>
__global__ __launch_bounds__(kThreads, 2) void gemm_kernel(const uint16_t* __restrict__ A,
                                                            const uint16_t* __restrict__ B,
                                                            uint16_t* __restrict__ C, float* __restrict__ P, int M,
                                                            int N, int K, int vec_a, int vec_b) {
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
    float H[2][2][16];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            acc[i][j] = (f16v){};
#pragma unroll
            for (int r = 0; r < 16; ++r) H[i][j][r] = 0.f;
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

    int ks_global = 0;   // index of the next 16-wide k step
    const int nks = (K + 15) / 16;
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
            if constexpr (MODE != kFp32) {
                const bool group_end = ((ks_global * 16) % GK == 0) || (ks_global == nks);
                if (group_end) {
                    if constexpr (MODE == kPartial) {
                        const int g = (ks_global * 16 - 1) / GK;
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
#pragma unroll
                        for (int i = 0; i < 2; ++i)
#pragma unroll
                            for (int j = 0; j < 2; ++j) fold_block<MODE, GN>(acc[i][j], H[i][j]);
                    }
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int j = 0; j < 2; ++j) acc[i][j] = (f16v){};
                }
            }
        }
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
                uint16_t h[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float v = MODE == kFp32 ? acc[i][j][4 * q + e] : H[i][j][4 * q + e];
                    _Float16 hv = (_Float16)v;
                    asm("" : "+v"(hv));
                    h[e] = __builtin_bit_cast(uint16_t, hv);
                }
                uint16_t* dst = C + m * (int64_t)N + n;
                if (n + 4 <= N && ((((uintptr_t)dst) & 7) == 0)) {
                    *reinterpret_cast<uint2*>(dst) =
                        make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16));
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

}  // namespace hbq_gemm

using namespace hbq_gemm;

namespace {

template <int MODE, int GK, int GN, bool BT>
void launch(const void* A, const void* B, void* C, float* P, int M, int N, int K, hipStream_t st) {
    dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
    int vec_a = (K % 8 == 0) && (((uintptr_t)A) % 16 == 0);
    int vec_b = (BT ? (K % 8 == 0) : (N % 8 == 0)) && (((uintptr_t)B) % 16 == 0);
    hipLaunchKernelGGL((gemm_kernel<MODE, GK, GN, BT>), grid, dim3(kThreads), 0, st, (const uint16_t*)A,
                       (const uint16_t*)B, (uint16_t*)C, P, M, N, K, vec_a, vec_b);
}

template <int MODE, int GK, bool BT>
int by_gn(int gn, const void* A, const void* B, void* C, int M, int N, int K, hipStream_t st) {
    switch (gn) {
        case 4: launch<MODE, GK, 4, BT>(A, B, C, nullptr, M, N, K, st); return 0;
        case 8: launch<MODE, GK, 8, BT>(A, B, C, nullptr, M, N, K, st); return 0;
        case 16: launch<MODE, GK, 16, BT>(A, B, C, nullptr, M, N, K, st); return 0;
        case 32: launch<MODE, GK, 32, BT>(A, B, C, nullptr, M, N, K, st); return 0;
    }
    return hbq_fail(HBQ_ERR_INVALID, "group_n must be one of {4,8,16,32}");
}

template <int MODE, bool BT>
int psum_dispatch(int gk, int gn, const void* A, const void* B, void* C, int M, int N, int K, hipStream_t st) {
    switch (gk) {
        case 64: return by_gn<MODE, 64, BT>(gn, A, B, C, M, N, K, st);
        case 128: return by_gn<MODE, 128, BT>(gn, A, B, C, M, N, K, st);
        case 256: return by_gn<MODE, 256, BT>(gn, A, B, C, M, N, K, st);
    }
    return hbq_fail(HBQ_ERR_INVALID, "group_k must be one of {64,128,256}");
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

}  // namespace

extern "C" {

int hbq_gemm_fp32_accum(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, int b_is_nk,
                        void* stream) {
    hbq_clear_error();
    if (int rc = check_shapes(A, B, C, M, N, K)) return rc;
    hipStream_t st = (hipStream_t)stream;
    if (M == 0 || N == 0) return 0;
    if (K == 0) return zero_output(C, M, N, st);
    if (b_is_nk) launch<kFp32, 16, 4, true>(A, B, C, nullptr, (int)M, (int)N, (int)K, st);
    else launch<kFp32, 16, 4, false>(A, B, C, nullptr, (int)M, (int)N, (int)K, st);
    return hbq_check_launch("gemm_fp32_accum");
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
#define GRP(G)                                                                                      \
    case G:                                                                                         \
        if (b_is_nk) launch<kGrouped, G, 4, true>(A, B, C, nullptr, (int)M, (int)N, (int)K, st);    \
        else launch<kGrouped, G, 4, false>(A, B, C, nullptr, (int)M, (int)N, (int)K, st);           \
        break;
    switch (group_k) { GRP(16) GRP(32) GRP(64) GRP(128) }
#undef GRP
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
    int rc;
    if (mode == kInt8)
        rc = b_is_nk ? psum_dispatch<kInt8, true>(gk, gn, A, B, C, (int)M, (int)N, (int)K, st)
                     : psum_dispatch<kInt8, false>(gk, gn, A, B, C, (int)M, (int)N, (int)K, st);
    else
        rc = b_is_nk ? psum_dispatch<kFp8, true>(gk, gn, A, B, C, (int)M, (int)N, (int)K, st)
                     : psum_dispatch<kFp8, false>(gk, gn, A, B, C, (int)M, (int)N, (int)K, st);
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

int hbq_gemm_group_partials(const void* A, const void* B, void* P, int64_t M, int64_t N, int64_t K, int group_k,
                            int b_is_nk, void* stream) {
    hbq_clear_error();
    if (group_k != 16 && group_k != 32 && group_k != 64 && group_k != 128 && group_k != 256)
        return hbq_fail(HBQ_ERR_INVALID, "group_k must be one of {16,32,64,128,256}");
    if (int rc = check_shapes(A, B, P, M, N, K)) return rc;
    if (M == 0 || N == 0 || K == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
#define GRP(G)                                                                                               \
    case G:                                                                                                  \
        if (b_is_nk) launch<kPartial, G, 4, true>(A, B, nullptr, (float*)P, (int)M, (int)N, (int)K, st);     \
        else launch<kPartial, G, 4, false>(A, B, nullptr, (float*)P, (int)M, (int)N, (int)K, st);            \
        break;
    switch (group_k) { GRP(16) GRP(32) GRP(64) GRP(128) GRP(256) }
#undef GRP
    return hbq_check_launch("gemm_group_partials");
}

}  // extern "C"
