// ABI version and thread-local error message of the C ABI.
#include "exl3_common.h"

namespace exl3 {

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

void clear_error() { g_err[0] = 0; }

}  // namespace exl3

extern "C" int exl3_abi_version(void) { return EXL3_ABI_VERSION; }

extern "C" const char* exl3_last_error(void) { return exl3::g_err; }
