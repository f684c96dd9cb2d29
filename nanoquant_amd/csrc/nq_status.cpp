// Status strings, per-thread error detail and launch checks of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "nq_common.h"

namespace nq {

static thread_local char g_last_error[512] = "";

int fail(int status, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return status;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(NQ_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return NQ_OK;
}

}  // namespace nq

extern "C" {

const char* nq_status_string(int status) {
    switch (status) {
        case NQ_OK: return "ok";
        case NQ_ERR_INVALID_ARGUMENT: return "invalid argument";
        case NQ_ERR_SHAPE: return "shape mismatch";
        case NQ_ERR_DTYPE: return "unsupported dtype";
        case NQ_ERR_ALIGNMENT: return "misaligned pointer";
        case NQ_ERR_WORKSPACE: return "workspace too small";
        case NQ_ERR_HIP: return "HIP runtime error";
        case NQ_ERR_UNSUPPORTED: return "unsupported configuration";
        default: return "unknown status";
    }
}

const char* nq_last_error_message(void) { return nq::g_last_error; }

int nq_version(void) { return 100; }

}  // extern "C"
