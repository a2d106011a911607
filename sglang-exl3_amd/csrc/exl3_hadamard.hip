// Row-wise 128-point Hadamard transform with optional fp16 scale vectors:
//   y[r][128c + j] = fp16( (H (x[r][128c..] (.) pre[128c..]))[j] * scale * post[128c + j] )
// One wave per 128-column chunk.  Stands in for exllamav3's had_r_128 as the
// reference calls it around its fat expert GEMM (src/sglang_exl3/exl3.py:1184,
// 1205, 1218, 1228) and backs transform_hadamard_fast
// (src/sglang_exl3/hadamard_cache.py:89-120).
#include "exl3_common.h"
#include "exl3_decode.h"

namespace exl3 {
namespace {

constexpr int HAD_THREADS = 256;

__device__ __forceinline__ float2 ld_h2f(const EXL3_GLOBAL __half* p) {
    const uint32_t u = *reinterpret_cast<const EXL3_GLOBAL uint32_t*>(p);
    const __half2 h = *reinterpret_cast<const __half2*>(&u);
    return make_float2(__low2float(h), __high2float(h));
}

__global__ __launch_bounds__(HAD_THREADS) void hadamard_rows_kernel(const __half* x, __half* y, const __half* pre,
                                                                    const __half* post, float scale,
                                                                    long long chunks, int cols) {
    const long long chunk = (long long)blockIdx.x * (HAD_THREADS / 64) + (threadIdx.x >> 6);
    if (chunk >= chunks) return;
    const int lane = threadIdx.x & 63;
    const int per_row = cols >> 7;
    const long long row = chunk / per_row;
    const int c = (int)(chunk - row * per_row) * 128 + 2 * lane;
    const size_t off = (size_t)row * cols + c;
    float2 v = ld_h2f(gptr(x) + off);
    if (pre) {
        const float2 s = ld_h2f(gptr(pre) + c);
        v.x *= s.x;
        v.y *= s.y;
    }
    float a = v.x, b = v.y;
    fwht128_pair_f(a, b, lane);
    a *= scale;
    b *= scale;
    if (post) {
        const float2 s = ld_h2f(gptr(post) + c);
        a *= s.x;
        b *= s.y;
    }
    const __half2 o = h2_rn(a, b);
    *reinterpret_cast<EXL3_GLOBAL uint32_t*>(gptr(y) + off) = *reinterpret_cast<const uint32_t*>(&o);
}

}  // namespace
}  // namespace exl3

using namespace exl3;

extern "C" int exl3_hadamard_rows(const uint16_t* x, uint16_t* y, const uint16_t* pre, const uint16_t* post,
                                  float scale, int rows, int cols, void* stream) {
    clear_error();
    EXL3_REQUIRE(rows >= 0 && cols > 0 && cols % 128 == 0, "exl3_hadamard_rows: rows=%d cols=%d (cols must be a "
                 "positive multiple of 128)", rows, cols);
    if (rows == 0) return EXL3_OK;
    EXL3_REQUIRE(x && y, "exl3_hadamard_rows: null pointer");
    EXL3_REQUIRE(aligned(x, 4) && aligned(y, 4) && aligned(pre, 4) && aligned(post, 4),
                 "exl3_hadamard_rows: misaligned pointer");
    const long long chunks = (long long)rows * (cols / 128);
    const long long blocks = (chunks + HAD_THREADS / 64 - 1) / (HAD_THREADS / 64);
    EXL3_REQUIRE(blocks <= 0x7fffffffLL, "exl3_hadamard_rows: %d x %d is too large", rows, cols);
    hadamard_rows_kernel<<<(unsigned)blocks, HAD_THREADS, 0, as_stream(stream)>>>(
        reinterpret_cast<const __half*>(x), reinterpret_cast<__half*>(y), reinterpret_cast<const __half*>(pre),
        reinterpret_cast<const __half*>(post), scale, chunks, cols);
    return launch_status("exl3_hadamard_rows launch");
}
