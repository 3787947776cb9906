// Library-level C ABI: version, thread-local error text, device properties.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "ss_common.hpp"

namespace ss {

static thread_local char g_err[1024] = {0};

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

int hip_fail(hipError_t e, const char *what) {
    set_error("%s: %s (%d)", what, hipGetErrorString(e), (int)e);
    return SS_ERR_HIP;
}

int device_cu_count() {
    static std::mutex mu;
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    std::lock_guard<std::mutex> lock(mu);
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
                hipSuccess ||
            n <= 0)
            n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

}  // namespace ss

extern "C" const char *ss_version(void) { return "sunshape_hip 0.1.0 gfx950"; }

extern "C" const char *ss_last_error(void) { return ss::g_err; }
