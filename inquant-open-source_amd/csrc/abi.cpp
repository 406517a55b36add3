// Error reporting and version query of the C ABI (host only).
#include <cstdarg>
#include <cstdio>

#include "../../include/inquant_hip.h"

namespace {
thread_local char g_last_error[512] = "";
}

int iq_fail(int status, const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return status;
}

extern "C" const char *iq_last_error(void) { return g_last_error; }

extern "C" int iq_abi_version(void) { return IQ_ABI_VERSION; }
