// Decode-level entry points: raw codebook lookups and un-rotated tile decode.
// They expose the device decode primitives every matmul kernel uses, so the
// bitstream, codebook and tile layout can be checked exhaustively on their own.
#include "exl3_common.h"
#include "exl3_decode.h"

namespace exl3 {
namespace {

template <int CB>
__global__ void decode_states_kernel(const uint16_t* __restrict__ st, int count, int rz,
                                     uint16_t* __restrict__ out) {
    const int i = (blockIdx.x * blockDim.x + threadIdx.x) * 2;
    if (i >= count) return;
    const uint32_t s0 = st[i];
    const uint32_t s1 = (i + 1 < count) ? st[i + 1] : 0u;
    const uint32_t v = rz ? decode2_rz<CB>(s0, s1) : decode2_rn<CB>(s0, s1);
    out[i] = (uint16_t)(v & 0xffffu);
    if (i + 1 < count) out[i + 1] = (uint16_t)(v >> 16);
}

template <int K, int CB, bool RZ>
__global__ void decode_tiles_kernel(const uint32_t* __restrict__ trellis, __half* __restrict__ W, int n,
                                    int total_groups) {
    const int gi = blockIdx.x * blockDim.x + threadIdx.x;
    if (gi >= total_groups) return;
    const int ntiles = n >> 4;
    const int tile = gi >> 3, q = gi & 7;
    const int kt = tile / ntiles, nt = tile - kt * ntiles;
    const uint32_t* tp = trellis + (size_t)tile * (8 * K);
    uint32_t buf[K + 1];
    buf[0] = tp[(K * q + 8 * K - 1) % (8 * K)];
#pragma unroll
    for (int w = 0; w < K; ++w) buf[1 + w] = tp[K * q + w];
    uint32_t frag[2][2][4];
    decode_group<K, CB, RZ>(buf, frag);
    unsigned short* Wu = reinterpret_cast<unsigned short*>(W);
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const uint32_t v = frag[c][h][p];
                const size_t col = (size_t)nt * 16 + q + 8 * c;
                const size_t r0 = (size_t)kt * 16 + 4 * h + kofs(2 * p);
                const size_t r1 = (size_t)kt * 16 + 4 * h + kofs(2 * p + 1);
                Wu[r0 * n + col] = (unsigned short)(v & 0xffffu);
                Wu[r1 * n + col] = (unsigned short)(v >> 16);
            }
}

template <int K>
int launch_tiles(int cb, int rz, const uint32_t* t, __half* W, int k, int n, hipStream_t st) {
    const int groups = (k / 16) * (n / 16) * 8;
    dim3 grid((groups + 255) / 256);
#define EXL3_DT(CBV, RZV) \
    if (cb == CBV && (rz != 0) == RZV) decode_tiles_kernel<K, CBV, RZV><<<grid, 256, 0, st>>>(t, W, n, groups);
    EXL3_DT(0, false) EXL3_DT(0, true) EXL3_DT(1, false) EXL3_DT(1, true) EXL3_DT(2, false) EXL3_DT(2, true)
#undef EXL3_DT
    return launch_status("exl3_decode_tiles launch");
}

}  // namespace
}  // namespace exl3

using namespace exl3;

extern "C" int exl3_decode_states(const uint16_t* states, int count, int codebook, int round_toward_zero,
                                  uint16_t* out, void* stream) {
    clear_error();
    EXL3_REQUIRE(states && out, "exl3_decode_states: null pointer");
    EXL3_REQUIRE(count >= 0, "exl3_decode_states: count=%d", count);
    EXL3_REQUIRE(codebook >= 0 && codebook <= 2, "exl3_decode_states: codebook=%d", codebook);
    if (count == 0) return EXL3_OK;
    hipStream_t st = as_stream(stream);
    dim3 grid(((count + 1) / 2 + 255) / 256);
    switch (codebook) {
        case 0: decode_states_kernel<0><<<grid, 256, 0, st>>>(states, count, round_toward_zero, out); break;
        case 1: decode_states_kernel<1><<<grid, 256, 0, st>>>(states, count, round_toward_zero, out); break;
        default: decode_states_kernel<2><<<grid, 256, 0, st>>>(states, count, round_toward_zero, out); break;
    }
    return launch_status("exl3_decode_states launch");
}

extern "C" int exl3_decode_tiles(const int16_t* trellis, uint16_t* W, int k, int n, int K, int codebook,
                                 int round_toward_zero, void* stream) {
    clear_error();
    EXL3_REQUIRE(trellis && W, "exl3_decode_tiles: null pointer");
    EXL3_REQUIRE(k > 0 && n > 0 && k % 16 == 0 && n % 16 == 0, "exl3_decode_tiles: k=%d n=%d", k, n);
    EXL3_REQUIRE(K >= 1 && K <= 8, "exl3_decode_tiles: K=%d outside 1..8", K);
    EXL3_REQUIRE(codebook >= 0 && codebook <= 2, "exl3_decode_tiles: codebook=%d", codebook);
    EXL3_REQUIRE(aligned(trellis, 4), "exl3_decode_tiles: misaligned trellis");
    const uint32_t* t = reinterpret_cast<const uint32_t*>(trellis);
    __half* w = reinterpret_cast<__half*>(W);
    hipStream_t st = as_stream(stream);
    const int rz = round_toward_zero;
    switch (K) {
        case 1: return launch_tiles<1>(codebook, rz, t, w, k, n, st);
        case 2: return launch_tiles<2>(codebook, rz, t, w, k, n, st);
        case 3: return launch_tiles<3>(codebook, rz, t, w, k, n, st);
        case 4: return launch_tiles<4>(codebook, rz, t, w, k, n, st);
        case 5: return launch_tiles<5>(codebook, rz, t, w, k, n, st);
        case 6: return launch_tiles<6>(codebook, rz, t, w, k, n, st);
        case 7: return launch_tiles<7>(codebook, rz, t, w, k, n, st);
        default: return launch_tiles<8>(codebook, rz, t, w, k, n, st);
    }
}
