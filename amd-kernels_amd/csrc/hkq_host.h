// hkq_host.h -- host-side helpers for the C-ABI entry points: argument checks
// that set a thread-local message and return hipErrorInvalidValue, and a
// launch-status check after each kernel launch.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hkq.h"

namespace hkq {
void set_error(const char* fmt, ...);
int fail_arg(const char* file, int line, const char* msg);
int cu_count();
}  // namespace hkq

#define HKQ_CHECK_ARG(cond, msg)                                     \
    do {                                                             \
        if (!(cond)) return ::hkq::fail_arg(__FILE__, __LINE__, msg); \
    } while (0)

#define HKQ_CHECK_ALIGN(ptr, a) \
    HKQ_CHECK_ARG((reinterpret_cast<uintptr_t>(ptr) % (a)) == 0, #ptr " must be " #a "-byte aligned")

// hipGetLastError after a launch: a bad configuration (grid too large, too much
// LDS) is reported here instead of silently dropping the work.
static inline int hkq_launch_status() {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) ::hkq::set_error("kernel launch failed: %s", hipGetErrorString(e));
    return (int)e;
}
