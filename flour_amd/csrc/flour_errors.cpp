// flour_errors.cpp — per-thread error message and version of libflour_hip.so.
#include <stdarg.h>
#include <stdio.h>

#include <string>

#include "flour_common.h"

namespace flour {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

int check_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return FLOUR_OK;
    set_error("%s: %s (%s)", what, hipGetErrorName(e), hipGetErrorString(e));
    return FLOUR_ERR_HIP;
}

}  // namespace flour

extern "C" const char* flour_hip_last_error(void) { return flour::g_last_error.c_str(); }

extern "C" const char* flour_hip_version(void) { return "flour_hip 0.1.0 (gfx950)"; }
