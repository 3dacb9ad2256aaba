// hkq_error.cpp -- thread-local error message of the C ABI and the device
// queries the launchers share.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>

#include "hkq_host.h"

namespace hkq {

static thread_local char g_msg[512] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
    va_end(ap);
}

int fail_arg(const char* file, int line, const char* msg) {
    const char* base = file;
    for (const char* c = file; *c; ++c)
        if (*c == '/') base = c + 1;
    set_error("%s (%s:%d)", msg, base, line);
    return (int)hipErrorInvalidValue;
}

// Compute units of the current device (cached per device; 0 if the query fails).
int cu_count() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
    if (dev < 64) {
        const int c = cache[dev].load(std::memory_order_relaxed);
        if (c > 0) return c;
    }
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 0;
    if (dev < 64) cache[dev].store(n, std::memory_order_relaxed);
    return n;
}

}  // namespace hkq

extern "C" const char* hkq_last_error(void) { return hkq::g_msg; }

extern "C" int hkq_version(void) { return (0 << 16) | 1; }
