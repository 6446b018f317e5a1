// capi.hip -- error reporting and library-level entry points of the C ABI.
#include "kvhp_internal.h"

#include <cstring>

namespace kvhp {

namespace {
thread_local char g_last_error[512] = {0};
}

void clear_error() { g_last_error[0] = 0; }

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_last_error, sizeof g_last_error, fmt, ap);
    va_end(ap);
}

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_last_error, sizeof g_last_error, fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return fail(KVHP_ERR_HIP, "%s: kernel launch failed: %s", what,
                    hipGetErrorString(e));
    return KVHP_OK;
}

}  // namespace kvhp

extern "C" const char* kvhp_last_error(void) { return kvhp::g_last_error; }

extern "C" int kvhp_abi_version(void) { return KVHP_ABI_VERSION; }
