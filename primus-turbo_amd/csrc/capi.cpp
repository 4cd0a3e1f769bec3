// Error state and version of the C ABI (include/primus_turbo_amd.h).
#include <cstdarg>
#include <cstdio>

#include "common.h"

namespace pta {

static thread_local char g_last_error[1024] = {0};

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

} // namespace pta

extern "C" const char *pta_last_error(void) { return pta::g_last_error; }

extern "C" int pta_abi_version(void) { return 5; }
