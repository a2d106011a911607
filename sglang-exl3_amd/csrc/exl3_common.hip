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

int allow_dynamic_lds(const void* kernel, size_t need, const char* what) {
    if (need <= 64 * 1024) return EXL3_OK;
    int dev = 0, max_lds = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess) {
        set_error("%s: cannot query the LDS limit", what);
        return EXL3_ERR_HIP;
    }
    hipFuncAttributes fa;
    if (hipFuncGetAttributes(&fa, kernel) != hipSuccess) {
        set_error("%s: cannot query kernel attributes", what);
        return EXL3_ERR_HIP;
    }
    const size_t avail = (size_t)max_lds > fa.sharedSizeBytes ? (size_t)max_lds - fa.sharedSizeBytes : 0;
    if (need > avail) {
        set_error("%s: needs %zu bytes of LDS, the device allows %zu", what, need, avail);
        return EXL3_ERR_UNSUPPORTED;
    }
    if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)need) != hipSuccess) {
        set_error("%s: cannot raise the dynamic LDS limit to %zu bytes", what, need);
        return EXL3_ERR_HIP;
    }
    return EXL3_OK;
}

}  // namespace exl3

extern "C" int exl3_abi_version(void) { return EXL3_ABI_VERSION; }

extern "C" const char* exl3_last_error(void) { return exl3::g_err; }
