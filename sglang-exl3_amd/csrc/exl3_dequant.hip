// exl3_dequant_trellis: whole-weight decode to fp16, bit-identical to the
// reference host dequant (csrc/bindings.cpp:15-100):
//   1. decode every tile with truncating fp16 rounding,
//   2. per 128x128 block: radix-2 FWHT of each row (strides 1..64), x norm,
//   3. FWHT of each column, then ((v * norm) * suh[r]) * svh[c] in fp32,
//   4. round to fp16 (nearest-even).
// One workgroup per 128x128 block; the block lives in LDS as fp32.
#include "exl3_common.h"
#include "exl3_decode.h"

namespace exl3 {
namespace {

constexpr int DQ_THREADS = 256;
constexpr int DQ_PITCH = 129;  // fp32 row pitch of the LDS block (bank spread)


template <int K, int CB>
__global__ __launch_bounds__(DQ_THREADS) void dequant_kernel(const uint32_t* __restrict__ trellis,
                                                             const __half* __restrict__ suh,
                                                             const __half* __restrict__ svh,
                                                             __half* __restrict__ W, int n) {
#pragma clang fp contract(off)
    __shared__ float M[128 * DQ_PITCH];
    const int bn = blockIdx.x, bk = blockIdx.y;
    const int ntiles = n >> 4;
    const int tid = threadIdx.x;

    // 1. decode the 64 tiles of the block: 512 groups of 32 values
    for (int gi = tid; gi < 512; gi += DQ_THREADS) {
        const int tile = gi >> 3, q = gi & 7;
        const int tk = tile >> 3, tn = tile & 7;
        const uint32_t* tp = trellis + ((size_t)(bk * 8 + tk) * ntiles + (bn * 8 + tn)) * (8 * K);
        uint32_t buf[K + 1];
        buf[0] = tp[(K * q + 8 * K - 1) % (8 * K)];
#pragma unroll
        for (int w = 0; w < K; ++w) buf[1 + w] = tp[K * q + w];
        uint32_t frag[2][2][4];
        decode_group<K, CB, true>(buf, frag);
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    const uint32_t v = frag[c][h][p];
                    const int col = tn * 16 + q + 8 * c;
                    const int r0 = tk * 16 + 4 * h + kofs(2 * p);
                    const int r1 = tk * 16 + 4 * h + kofs(2 * p + 1);
                    M[r0 * DQ_PITCH + col] = __half2float(__ushort_as_half((unsigned short)(v & 0xffffu)));
                    M[r1 * DQ_PITCH + col] = __half2float(__ushort_as_half((unsigned short)(v >> 16)));
                }
    }
    __syncthreads();

    const int wave = tid >> 6, lane = tid & 63;
    // 2. row pass
    for (int r = wave; r < 128; r += DQ_THREADS / 64) {
        float a = M[r * DQ_PITCH + 2 * lane], b = M[r * DQ_PITCH + 2 * lane + 1];
        fwht128_pair_f(a, b, lane);
        M[r * DQ_PITCH + 2 * lane] = a * kHadNorm;
        M[r * DQ_PITCH + 2 * lane + 1] = b * kHadNorm;
    }
    __syncthreads();

    // 3. column pass with the sign scales
    const int r0 = bk * 128, c0 = bn * 128;
    const float su0 = __half2float(suh[r0 + 2 * lane]);
    const float su1 = __half2float(suh[r0 + 2 * lane + 1]);
    for (int c = wave; c < 128; c += DQ_THREADS / 64) {
        float a = M[(2 * lane) * DQ_PITCH + c], b = M[(2 * lane + 1) * DQ_PITCH + c];
        fwht128_pair_f(a, b, lane);
        const float sv = __half2float(svh[c0 + c]);
        float va = a * kHadNorm;
        va = va * su0;
        va = va * sv;
        float vb = b * kHadNorm;
        vb = vb * su1;
        vb = vb * sv;
        M[(2 * lane) * DQ_PITCH + c] = va;
        M[(2 * lane + 1) * DQ_PITCH + c] = vb;
    }
    __syncthreads();

    // 4. store fp16 rows (16 B per thread)
    for (int idx = tid; idx < 128 * 16; idx += DQ_THREADS) {
        const int r = idx >> 4, c8 = (idx & 15) * 8;
        uint32_t o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            __half lo = __float2half_rn(M[r * DQ_PITCH + c8 + 2 * j]);
            __half hi = __float2half_rn(M[r * DQ_PITCH + c8 + 2 * j + 1]);
            o[j] = (uint32_t)__half_as_ushort(lo) | ((uint32_t)__half_as_ushort(hi) << 16);
        }
        *reinterpret_cast<uint4*>(W + (size_t)(r0 + r) * (size_t)(ntiles * 16) + c0 + c8) =
            make_uint4(o[0], o[1], o[2], o[3]);
    }
}

template <int K>
int launch_dequant_k(int cb, const uint32_t* t, const __half* su, const __half* sv, __half* W, int k, int n,
                     hipStream_t st) {
    dim3 grid(n / 128, k / 128);
    switch (cb) {
        case 0: dequant_kernel<K, 0><<<grid, DQ_THREADS, 0, st>>>(t, su, sv, W, n); break;
        case 1: dequant_kernel<K, 1><<<grid, DQ_THREADS, 0, st>>>(t, su, sv, W, n); break;
        default: dequant_kernel<K, 2><<<grid, DQ_THREADS, 0, st>>>(t, su, sv, W, n); break;
    }
    return launch_status("exl3_dequant_trellis launch");
}

}  // namespace
}  // namespace exl3

extern "C" int exl3_dequant_trellis(const int16_t* trellis, const uint16_t* suh, const uint16_t* svh,
                                    uint16_t* W, int k, int n, int K, int codebook, void* stream) {
    using namespace exl3;
    clear_error();
    EXL3_REQUIRE(trellis && suh && svh && W, "exl3_dequant_trellis: null pointer");
    EXL3_REQUIRE(k > 0 && n > 0 && k % 128 == 0 && n % 128 == 0,
                 "exl3_dequant_trellis: k=%d n=%d must be positive multiples of 128", k, n);
    EXL3_REQUIRE(K >= 1 && K <= 8, "exl3_dequant_trellis: K=%d outside 1..8", K);
    EXL3_REQUIRE(codebook >= 0 && codebook <= 2, "exl3_dequant_trellis: codebook=%d", codebook);
    EXL3_REQUIRE(aligned(trellis, 4) && aligned(W, 16), "exl3_dequant_trellis: misaligned pointer");
    const uint32_t* t = reinterpret_cast<const uint32_t*>(trellis);
    const __half* su = reinterpret_cast<const __half*>(suh);
    const __half* sv = reinterpret_cast<const __half*>(svh);
    __half* w = reinterpret_cast<__half*>(W);
    hipStream_t st = as_stream(stream);
    switch (K) {
        case 1: return launch_dequant_k<1>(codebook, t, su, sv, w, k, n, st);
        case 2: return launch_dequant_k<2>(codebook, t, su, sv, w, k, n, st);
        case 3: return launch_dequant_k<3>(codebook, t, su, sv, w, k, n, st);
        case 4: return launch_dequant_k<4>(codebook, t, su, sv, w, k, n, st);
        case 5: return launch_dequant_k<5>(codebook, t, su, sv, w, k, n, st);
        case 6: return launch_dequant_k<6>(codebook, t, su, sv, w, k, n, st);
        case 7: return launch_dequant_k<7>(codebook, t, su, sv, w, k, n, st);
        default: return launch_dequant_k<8>(codebook, t, su, sv, w, k, n, st);
    }
}
