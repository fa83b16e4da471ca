// flour_errors.cpp — per-thread error message and version of libflour_hip.so.
#include <stdarg.h>
#include <stdio.h>

#include "flour_common.h"

namespace flour {

// A fixed buffer, so that recording an error never allocates (it may report a failed
// allocation); longer messages are truncated.
static thread_local char g_last_error[512];

void set_error(const char* fmt, ...) noexcept {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
}

void clear_error() noexcept { g_last_error[0] = '\0'; }

int check_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return FLOUR_OK;
    set_error("%s: %s (%s)", what, hipGetErrorName(e), hipGetErrorString(e));
    return FLOUR_ERR_HIP;
}

}  // namespace flour

extern "C" const char* flour_hip_last_error(void) { return flour::g_last_error; }

extern "C" const char* flour_hip_version(void) { return "flour_hip 0.1.0 (gfx950)"; }
