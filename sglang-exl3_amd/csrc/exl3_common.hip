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

extern "C" int exl3_workspace_status(void* workspace, size_t workspace_bytes, int32_t* status_out, void* stream) {
    using namespace exl3;
    clear_error();
    EXL3_REQUIRE(workspace && status_out, "exl3_workspace_status: null pointer");
    EXL3_REQUIRE(workspace_bytes >= kWsCounterBytes, "exl3_workspace_status: workspace of %zu bytes has no status word",
                 workspace_bytes);
    hipStream_t st = as_stream(stream);
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess) {
        set_error("exl3_workspace_status: cannot query the stream's capture state");
        return EXL3_ERR_HIP;
    }
    EXL3_REQUIRE(cs == hipStreamCaptureStatusNone, "exl3_workspace_status: cannot run during graph capture");
    int32_t* word = reinterpret_cast<int32_t*>(workspace) + kWsStatusIndex;
    int32_t host = 0;
    static const int32_t zero = 0;
    if (hipMemcpyAsync(&host, word, sizeof(int32_t), hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess) {
        set_error("exl3_workspace_status: reading the status word failed");
        return EXL3_ERR_HIP;
    }
    if (host != 0 && (hipMemcpyAsync(word, &zero, sizeof(int32_t), hipMemcpyHostToDevice, st) != hipSuccess ||
                      hipStreamSynchronize(st) != hipSuccess)) {
        set_error("exl3_workspace_status: clearing the status word failed");
        return EXL3_ERR_HIP;
    }
    *status_out = host;
    return EXL3_OK;
}
