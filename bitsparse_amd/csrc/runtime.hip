// Error reporting and version entry points of libbitsparse_hip.so.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "bs_host.h"

namespace bs {

static thread_local char g_err[512];

int set_error(int code, const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { g_err[0] = '\0'; }

}  // namespace bs

extern "C" const char* bs_last_error(void) { return bs::g_err; }

extern "C" int bs_abi_version(void) { return 3; }
