// Entry of the table-driven HBQ kernel (hbq_fast.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "quant_common.h"

// Runs the table-driven kernel when the configuration and layout allow it.
// Returns 1 when launched, 0 when the caller must use the generic kernel, and
// a negative HBQ_ERR_* code on a HIP error (message already recorded).
// causal_t > 0: x is [rows / causal_t, causal_t, causal_t] attention weights quantized
// in place (y == x), the blocks entirely above the diagonal (zero) left untouched.
int hbq_fast_try(const void* x, void* y, void* l1, void* l2i, void* sch, void* codes, int64_t rows, int64_t cols,
                 int dtype, int block, int mbit, int l2b, int l2_sc_bit, int scheme, const hbq::HbqParams& hp,
                 hipStream_t st, int64_t causal_t = 0);

namespace hbq {
// Where the table kernel's input comes from: memory (kSrcX), or computed on the fly by
// the pass that would have produced it (its output never written): the RMSNorm apply
// step R(w[col] * R(R32(a * rs[row]))) (kSrcRms: a = the residual-stream sum, b = w),
// or the SiLU product R(R(silu(a)) * b) (kSrcSilu: a = gate, b = up).
enum FastSrcKind : int { kSrcX = 0, kSrcRms = 1, kSrcSilu = 2 };
struct FastSrc {
    int kind;
    const uint16_t* a;
    const uint16_t* b;
    const float* rs;
};
}  // namespace hbq

// hbq_fast_try on a computed input (kSrcRms / kSrcSilu): y = the quantizer's output only.
// Returns 1 when launched, 0 when the configuration is outside the fused kernels (act
// formats: E2M2, one scheme, block 128), a negative HBQ_ERR_* code on a HIP error.
int hbq_fast_try_src(const hbq::FastSrc& src, void* y, int64_t rows, int64_t cols, int dtype, int block, int mbit,
                     int l2b, int l2_sc_bit, int scheme, const hbq::HbqParams& hp, hipStream_t st);
