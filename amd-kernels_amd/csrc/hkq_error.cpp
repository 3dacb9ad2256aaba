// hkq_error.cpp -- thread-local error message of the C ABI.
#include <stdarg.h>
#include <stdio.h>

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

}  // namespace hkq

extern "C" const char* hkq_last_error(void) { return hkq::g_msg; }

extern "C" int hkq_version(void) { return (0 << 16) | 1; }
