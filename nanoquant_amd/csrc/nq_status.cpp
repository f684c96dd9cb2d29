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

// ----------------------------------------------------------------------------- measurement aid

namespace nq {
namespace {
__global__ void wall_clock_kernel(uint64_t* dst) { *dst = wall_clock64(); }
}  // namespace
}  // namespace nq

extern "C" {

int nq_timestamp(uint64_t* dst, nq_stream_t stream) {
    if (!dst) return nq::fail(NQ_ERR_INVALID_ARGUMENT, "nq_timestamp: null pointer");
    nq::wall_clock_kernel<<<1, 1, 0, nq::as_stream(stream)>>>(dst);
    return nq::check_launch("nq_timestamp");
}

int64_t nq_wall_clock_hz(void) {
    int dev = 0, khz = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess) return 0;
    return static_cast<int64_t>(khz) * 1000;
}

}  // extern "C"
