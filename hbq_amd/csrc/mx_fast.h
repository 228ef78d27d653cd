// Entry of the table-driven MXFP / NVFP kernel (mx_fast.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "quant_common.h"

// Runs the table-driven kernel when the configuration and layout allow it
// (fp16, block 16 or 32, whole blocks per row, no per-tensor scale).  Returns 1
// when launched, 0 when the caller must use the generic kernel, and a negative
// HBQ_ERR_* code on a HIP error (message already recorded).
int hbq_mx_fast_try(const void* x, void* y, void* scales, void* codes, int64_t rows, int64_t cols, int dtype,
                    int block, int mbit, const hbq::MxParams& p, hipStream_t st);
