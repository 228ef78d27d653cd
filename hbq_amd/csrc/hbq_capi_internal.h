// Error reporting shared by the C-ABI entry points.
#pragma once
#include <hip/hip_runtime.h>

#define HBQ_OK 0
#define HBQ_ERR_INVALID 1       // argument check failed (the reference raises RuntimeError/ValueError)
#define HBQ_ERR_UNSUPPORTED 2   // configuration outside what the GPU path implements
#define HBQ_ERR_HIP 3           // HIP runtime / launch error

int hbq_fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void hbq_clear_error();
int hbq_check_launch(const char* what);
