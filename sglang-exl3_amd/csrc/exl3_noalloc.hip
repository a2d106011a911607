// exl3_gemv_noalloc: exl3_gemv for callers that cannot allocate device memory
// (code under HIP graph capture, serving loops, harnesses that forbid
// hipMalloc).  The split-k counters, fixed-point accumulators and partial sums
// live in a file-scope device array of EXL3_NOALLOC_SCRATCH_BYTES instead of a
// caller workspace.  Every call on one GPU shares that GPU's array: calls
// that overlap on one GPU (several streams, several threads) race.
#include <mutex>

#include "exl3_common.h"

namespace exl3 {
namespace {

static_assert(EXL3_NOALLOC_SCRATCH_BYTES >= kWsScratchOffset, "scratch must hold the zeroed workspace regions");

// One copy per GPU, held until the process ends.  Host code never uses this
// name as an address: it only stands in for the symbol; the device address
// comes from hipGetSymbolAddress (kept per device below).
__device__ __align__(256) unsigned char scratch[EXL3_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices];  // device address of `scratch` on each device (null: not set up yet)

// Zero the counter and accumulator regions (vector stores; no memset node,
// so a first call under graph capture records a plain kernel).
__global__ __launch_bounds__(256) void clear_zero_regions_kernel(uint4* p, size_t n16) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x)
        p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// Device address of this device's scratch; the first call on a device looks
// the symbol up and enqueues the clear of its zeroed regions on `st`.
int scratch_for_device(hipStream_t st, void** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        set_error("exl3_gemv_noalloc: no current HIP device (or device index above %d)", kMaxDevices - 1);
        return EXL3_ERR_HIP;
    }
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            set_error("exl3_gemv_noalloc: hipGetSymbolAddress of the scratch array failed on device %d: %s", dev,
                      hipGetErrorString(e));
            return EXL3_ERR_HIP;
        }
        const size_t n16 = kWsScratchOffset / 16;
        clear_zero_regions_kernel<<<256, 256, 0, st>>>(reinterpret_cast<uint4*>(p), n16);
        const int rc = launch_status("exl3_gemv_noalloc scratch clear");
        if (rc) return rc;
        g_ptr[dev] = p;
    }
    *out = g_ptr[dev];
    return EXL3_OK;
}

}  // namespace
}  // namespace exl3

using namespace exl3;

extern "C" int exl3_gemv_noalloc(const uint16_t* x, const int16_t* trellis, const uint16_t* suh,
                                 const uint16_t* svh, uint16_t* y, int m, int k, int n, int K, int codebook,
                                 void* stream) {
    clear_error();
    // every argument is checked before the device is touched
    EXL3_REQUIRE(m >= 1 && m <= 64, "exl3_gemv_noalloc: m=%d outside 1..64", m);
    EXL3_REQUIRE(k > 0 && n > 0 && k % 128 == 0 && n % 128 == 0,
                 "exl3_gemv_noalloc: k=%d n=%d must be positive multiples of 128", k, n);
    EXL3_REQUIRE(K >= 1 && K <= 8, "exl3_gemv_noalloc: K=%d outside 1..8", K);
    EXL3_REQUIRE(codebook >= 0 && codebook <= 2, "exl3_gemv_noalloc: codebook=%d outside 0..2", codebook);
    EXL3_REQUIRE(x && trellis && suh && svh && y, "exl3_gemv_noalloc: null pointer");
    const size_t need = exl3_gemv_workspace_size(m, k, n, K, 1);
    EXL3_REQUIRE_CODE(need <= EXL3_NOALLOC_SCRATCH_BYTES, EXL3_ERR_UNSUPPORTED,
                      "exl3_gemv_noalloc: m=%d k=%d n=%d needs %zu bytes of scratch, above the fixed %zu "
                      "(use exl3_gemv with a workspace)",
                      m, k, n, need, (size_t)EXL3_NOALLOC_SCRATCH_BYTES);
    hipStream_t st = as_stream(stream);
    void* ws = nullptr;
    int rc = scratch_for_device(st, &ws);
    if (rc) return rc;
    return exl3_gemv(x, trellis, suh, svh, y, m, k, n, K, codebook, ws, EXL3_NOALLOC_SCRATCH_BYTES, stream);
}
