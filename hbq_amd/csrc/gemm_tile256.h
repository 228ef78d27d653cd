// The 256x256-tile block-quant GEMM (gemm_tile256.hip): W[N,K] operand layout,
// K a multiple of 64, N a multiple of 8, 16-byte aligned operands.
#pragma once
#include <hip/hip_runtime.h>

namespace hbq_gemm {

// Launches the 256x256 kernel for (mode, group_n) when the shape and layout
// allow it and returns 1; returns 0 (nothing launched) otherwise.
int launch_tile256(int mode, int gn, const void* A, const void* B, void* C, float* P, int M, int N, int K, int gk,
                   int b_is_nk, hipStream_t st);

// Split K for fp32 accumulation: the number of K ranges worth running for this shape
// (1: none), and the launch (splits x M x N fp32 partials in ws, then their sum in
// split order rounded to fp16); returns 0 when the layout does not allow it.
int splitk_fp32_splits(int M, int N, int K);
int launch_splitk_fp32(const void* A, const void* W, void* C, float* ws, int M, int N, int K, int splits,
                       hipStream_t st);

// fp32 accumulation over `batches` independent problems C_z = A_z W_{z / wgroup}^T
// (element strides sA, sW, sC between them; row stride ldc of C) in one launch; 0 when
// the layout does not allow it.
int launch_batched_fp32(const void* A, const void* W, void* C, int batches, int M, int N, int K, int64_t sA,
                        int64_t sW, int64_t sC, int wgroup, int64_t ldc, hipStream_t st);

}  // namespace hbq_gemm
