// Error state and small utilities of the C ABI (declared in include/hbq_amd.h).
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "hbq_capi_internal.h"

static thread_local char g_err[512];

int hbq_fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

void hbq_clear_error() { g_err[0] = '\0'; }

int hbq_check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hbq_fail(HBQ_ERR_HIP, "%s kernel failed: %s", what, hipGetErrorString(e));
    return HBQ_OK;
}

extern "C" {

const char* hbq_last_error(void) { return g_err; }

int hbq_abi_version(void) { return 2; }

}
