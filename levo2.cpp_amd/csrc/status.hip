// Per-thread last-error message of the C ABI (the pattern of the reference's
// cantor_engine_last_error, src/cantor-abi.cpp:58-82).
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <map>
#include <mutex>
#include <set>
#include <string>
#include <utility>

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

int allow_dynamic_lds(const void * kernel, int bytes, const char * what) {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) {
        set_error("%s: cannot query the current device", what);
        return LEVO_HIP_ERR_RUNTIME;
    }
    static std::mutex mu;
    static std::set<std::pair<const void *, int>> done;  // (kernel, device) pairs already raised
    std::lock_guard<std::mutex> lock(mu);
    if (done.count({kernel, device})) return LEVO_HIP_OK;
    if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) != hipSuccess) {
        set_error("%s: cannot raise the LDS limit", what);
        return LEVO_HIP_ERR_RUNTIME;
    }
    done.insert({kernel, device});
    return LEVO_HIP_OK;
}

int device_cu_count() {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0) return 0;
    static std::mutex mu;
    static std::map<int, int> counts;
    std::lock_guard<std::mutex> lock(mu);
    const auto it = counts.find(device);
    if (it != counts.end()) return it->second;
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) n = 0;
    counts[device] = n;
    return n;
}

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
