// Per-thread last-error message of the C ABI (the pattern of the reference's
// cantor_engine_last_error, src/cantor-abi.cpp:58-82).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "common.hpp"

namespace levo_hip {
namespace {
thread_local std::string g_last_error;
}

void set_error(const char * fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

int launch_status(const char * what) {
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
        set_error("%s: HIP launch failed: %s", what, hipGetErrorString(err));
        return LEVO_HIP_ERR_RUNTIME;
    }
    return LEVO_HIP_OK;
}

}  // namespace levo_hip

extern "C" const char * levo_hip_last_error(void) { return levo_hip::g_last_error.c_str(); }

extern "C" int levo_hip_abi_version(void) { return LEVO_HIP_ABI_VERSION; }
