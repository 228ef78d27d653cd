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
