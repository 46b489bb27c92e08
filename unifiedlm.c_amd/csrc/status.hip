// Error reporting shared by every entry point of libulm_fm.so.
#include <stdarg.h>
#include <stdio.h>

#include "ulm_common.h"

namespace ulm {

static thread_local char g_last_error[512] = "";

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(ULM_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
    return ULM_OK;
}

}  // namespace ulm

extern "C" int ulm_abi_version(void) { return 3; }

extern "C" const char *ulm_last_error(void) { return ulm::g_last_error; }
