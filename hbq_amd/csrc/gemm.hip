// placeholder, replaced by the MFMA GEMM kernels
#include <hip/hip_runtime.h>
