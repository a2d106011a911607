// Row-wise 128-point Hadamard transform with optional fp16 scale vectors:
//   y[r][128c + j] = fp16( (H (x[r][128c..] (.) pre[128c..]))[j] * scale * post[128c + j] )
// One wave per 128-column chunk.  Stands in for exllamav3's had_r_128 as the
// reference calls it around its fat expert GEMM (src/sglang_exl3/exl3.py:1184,
// 1205, 1218, 1228).  exl3_hadamard_fast below backs transform_hadamard_fast
// (src/sglang_exl3/hadamard_cache.py:88-120) in fp16, bf16 and fp32.
#include <hip/hip_bf16.h>

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

// transform_hadamard_fast in the caller's dtype T: the reference multiplies
// each 128-block by a Sylvester matrix of +-T(1/sqrt(128)) in T (products
// exact, fp32 accumulation), rounds to T, then multiplies by suh converted
// to T and rounds again (src/sglang_exl3/hadamard_cache.py:103-118).  Here
// the block sum runs in fp32 in FWHT order and is scaled once by the same
// T-rounded factor; the two T roundings are the reference's.
struct IoF16 {
    typedef __half T;
    static __device__ __forceinline__ float2 ld(const T* p) { return ld_h2f(gptr(p)); }
    static __device__ __forceinline__ float rt(float v) { return __half2float(__float2half_rn(v)); }
    static __device__ __forceinline__ void st(T* p, float a, float b) {
        const __half2 o = h2_rn(a, b);
        *reinterpret_cast<EXL3_GLOBAL uint32_t*>(gptr(p)) = *reinterpret_cast<const uint32_t*>(&o);
    }
};
struct IoBf16 {
    typedef __hip_bfloat16 T;
    static __device__ __forceinline__ float2 ld(const T* p) {
        const uint32_t u = *reinterpret_cast<const EXL3_GLOBAL uint32_t*>(gptr(p));
        return make_float2(__uint_as_float(u << 16), __uint_as_float(u & 0xffff0000u));
    }
    static __device__ __forceinline__ float rt(float v) { return __bfloat162float(__float2bfloat16(v)); }
    static __device__ __forceinline__ void st(T* p, float a, float b) {
        const uint32_t lo = __bfloat16_as_ushort(__float2bfloat16(a));
        const uint32_t hi = __bfloat16_as_ushort(__float2bfloat16(b));
        *reinterpret_cast<EXL3_GLOBAL uint32_t*>(gptr(p)) = lo | (hi << 16);
    }
};
struct IoF32 {
    typedef float T;
    static __device__ __forceinline__ float2 ld(const T* p) {
        const uint64_t u = *reinterpret_cast<const EXL3_GLOBAL uint64_t*>(gptr(p));
        return make_float2(__uint_as_float((uint32_t)u), __uint_as_float((uint32_t)(u >> 32)));
    }
    static __device__ __forceinline__ float rt(float v) { return v; }
    static __device__ __forceinline__ void st(T* p, float a, float b) {
        *reinterpret_cast<EXL3_GLOBAL uint64_t*>(gptr(p)) =
            (uint64_t)__float_as_uint(a) | ((uint64_t)__float_as_uint(b) << 32);
    }
};

template <typename Io>
__global__ __launch_bounds__(HAD_THREADS) void hadamard_fast_kernel(const typename Io::T* x, typename Io::T* y,
                                                                    const typename Io::T* post, float h,
                                                                    long long chunks, int cols) {
    const long long chunk = (long long)blockIdx.x * (HAD_THREADS / 64) + (threadIdx.x >> 6);
    if (chunk >= chunks) return;
    const int lane = threadIdx.x & 63;
    const int per_row = cols >> 7;
    const long long row = chunk / per_row;
    const int c = (int)(chunk - row * per_row) * 128 + 2 * lane;
    const size_t off = (size_t)row * cols + c;
    const float2 v = Io::ld(x + off);
    float a = v.x, b = v.y;
    fwht128_pair_f(a, b, lane);
    a = Io::rt(a * h);
    b = Io::rt(b * h);
    if (post) {
        const float2 s = Io::ld(post + c);
        a *= s.x;
        b *= s.y;
    }
    Io::st(y + off, a, b);
}

template <typename Io>
void launch_hadamard_fast(const void* x, void* y, const void* post, float h, long long chunks, long long blocks,
                          int cols, hipStream_t st) {
    typedef typename Io::T T;
    hadamard_fast_kernel<Io><<<(unsigned)blocks, HAD_THREADS, 0, st>>>(
        reinterpret_cast<const T*>(x), reinterpret_cast<T*>(y), reinterpret_cast<const T*>(post), h, chunks, cols);
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

extern "C" int exl3_hadamard_fast(const void* x, void* y, const void* post, int rows, int cols, int dtype,
                                  void* stream) {
    clear_error();
    EXL3_REQUIRE(dtype >= EXL3_DTYPE_F16 && dtype <= EXL3_DTYPE_F32, "exl3_hadamard_fast: dtype=%d (0 fp16, 1 bf16, "
                 "2 fp32)", dtype);
    EXL3_REQUIRE(rows >= 0 && cols > 0 && cols % 128 == 0, "exl3_hadamard_fast: rows=%d cols=%d (cols must be a "
                 "positive multiple of 128)", rows, cols);
    if (rows == 0) return EXL3_OK;
    EXL3_REQUIRE(x && y, "exl3_hadamard_fast: null pointer");
    const size_t al = dtype == EXL3_DTYPE_F32 ? 8 : 4;  // one lane moves two elements
    EXL3_REQUIRE(aligned(x, al) && aligned(y, al) && aligned(post, al), "exl3_hadamard_fast: misaligned pointer");
    const long long chunks = (long long)rows * (cols / 128);
    const long long blocks = (chunks + HAD_THREADS / 64 - 1) / (HAD_THREADS / 64);
    EXL3_REQUIRE(blocks <= 0x7fffffffLL, "exl3_hadamard_fast: %d x %d is too large", rows, cols);
    // +-1/sqrt(128) as the reference's matrix holds it: fp32, then rounded to
    // the dtype (181 / 2048 in fp16 and bf16 alike)
    const float h32 = 0.0883883461356163f, h16 = 181.0f / 2048.0f;
    const hipStream_t st = as_stream(stream);
    if (dtype == EXL3_DTYPE_F16) launch_hadamard_fast<IoF16>(x, y, post, h16, chunks, blocks, cols, st);
    else if (dtype == EXL3_DTYPE_BF16) launch_hadamard_fast<IoBf16>(x, y, post, h16, chunks, blocks, cols, st);
    else launch_hadamard_fast<IoF32>(x, y, post, h32, chunks, blocks, cols, st);
    return launch_status("exl3_hadamard_fast launch");
}
