// Library-level C ABI: version, status strings, thread-local error text.
#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "kf_common.h"

namespace kf {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

int hip_failure(hipError_t err, const char* what) {
    set_error("%s: %s (%s)", what, hipGetErrorString(err), hipGetErrorName(err));
    return KF_E_HIP;
}

int device_cu_count() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0)
            cus = 256;
        cached[dev] = cus;
    }
    return cached[dev];
}

}  // namespace kf

extern "C" {

int kf_abi_version(void) { return KF_ABI_VERSION; }

const char* kf_status_string(int status) {
    switch (status) {
        case KF_OK: return "KF_OK";
        case KF_E_INVALID: return "KF_E_INVALID";
        case KF_E_UNSUPPORTED: return "KF_E_UNSUPPORTED";
        case KF_E_WORKSPACE: return "KF_E_WORKSPACE";
        case KF_E_HIP: return "KF_E_HIP";
        case KF_E_INCOMPLETE: return "KF_E_INCOMPLETE";
        default: return "KF_E_UNKNOWN";
    }
}

const char* kf_last_error(void) { return kf::g_last_error; }

}  // extern "C"
