// Shared host-side helpers of the C ABI: error reporting and launch checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "../../include/sglang_exl3_amd.h"

namespace exl3 {

// Thread-local message behind exl3_last_error().
void set_error(const char* fmt, ...);
void clear_error();

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Check the launch just enqueued; converts a HIP error into EXL3_ERR_HIP.
inline int launch_status(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: %s", what, hipGetErrorString(e));
        return EXL3_ERR_HIP;
    }
    return EXL3_OK;
}

// Workspace layout shared by every kernel that needs one:
//   [0, 256 KiB)          int counters of the split-k hand-offs;
//   [256 KiB, 4.25 MiB)   64-bit fixed-point output accumulators of the
//                         balanced GEMV;
//   [4.25 MiB, ...)       per-call scratch (partials, staged rows, ...).
// The first two regions are zero between calls (the caller zeroes the buffer
// once; every kernel resets what it used).  Scratch starts at a fixed offset,
// so no call's scratch ever overlaps the zeroed regions.
constexpr size_t kWsCounterBytes = 256 * 1024;
// Counters a call may use; the last 64 ints of the region are kept out of
// counter use and hold the bounded-wait status word (kWsStatusIndex).
constexpr size_t kWsMaxCounters = kWsCounterBytes / sizeof(int) - 64;
// Status word (int index into the counter region): a kernel whose bounded
// wait gave up ORs its EXL3_WAIT_* bit in; exl3_workspace_status reads and
// clears it.
constexpr size_t kWsStatusIndex = kWsCounterBytes / sizeof(int) - 1;

constexpr size_t kWsAccOffset = kWsCounterBytes;
constexpr size_t kWsAccBytes = 4 * 1024 * 1024;
constexpr size_t kWsScratchOffset = kWsAccOffset + kWsAccBytes;

// Polls a bounded wait makes before it gives up (each poll is followed by
// ~0.2 us of s_sleep, so the default is ~0.25 s, far beyond any hand-off
// inside one launch).  Env EXL3_WAIT_POLLS overrides it (tests set 0 to
// make a wait give up from the host), clamped to [0, 2^24].
constexpr int kWaitPolls = 1 << 20;

// LDS a gfx950 workgroup may allocate.
constexpr size_t kMaxLds = 160 * 1024;

// Let `kernel` take up to `need` bytes of dynamic LDS (the runtime default cap
// is 64 KB).  Checks the device limit and the kernel's static LDS; returns
// EXL3_OK or an error with a message.
int allow_dynamic_lds(const void* kernel, size_t need, const char* what);

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Integer value of environment variable `name` (tuning overrides, read per
// call), or `dflt` when it is unset or empty.
inline int env_int(const char* name, int dflt) {
    const char* v = getenv(name);
    if (!v || !*v) return dflt;
    return atoi(v);
}

inline int wait_polls() {
    const int v = env_int("EXL3_WAIT_POLLS", kWaitPolls);
    return v < 0 ? 0 : (v > (1 << 24) ? (1 << 24) : v);
}

// exl3_gemm: GEMV kernels up to this many rows for outputs narrower than
// 12288 columns, kGemmGemvRowsWide from 12288 and one row fewer from 24576;
// the MFMA GEMM above (gemm_gemv_rows(n), env override).
constexpr int kGemmGemvRows = 12;
constexpr int kGemmGemvRowsWide = 8;
int gemm_gemv_rows(int n);

}  // namespace exl3

#define EXL3_REQUIRE(cond, ...)                  \
    do {                                         \
        if (!(cond)) {                           \
            exl3::set_error(__VA_ARGS__);        \
            return EXL3_ERR_ARG;                 \
        }                                        \
    } while (0)

#define EXL3_REQUIRE_CODE(cond, code, ...)       \
    do {                                         \
        if (!(cond)) {                           \
            exl3::set_error(__VA_ARGS__);        \
            return (code);                       \
        }                                        \
    } while (0)
