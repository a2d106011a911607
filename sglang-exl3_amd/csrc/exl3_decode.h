// EXL3 trellis decode primitives for CDNA4 (gfx950).
//
// Format (the reference's, restated): a 16x16 weight tile is a tail-biting
// bitstream of 256*K bits held as 8*K little-endian uint32 words.  Value t of
// the tile is the 16-bit window ending at stream bit (t+1)*K, bits taken
// MSB-first across words (csrc/exl3_dequant.cuh:110-135,
// csrc/quant/exl3_dq.cuh:15-30).  Value t lands at
//   k = 2(l%4) + (j&1) + 8((j>>1)&1),  n = l/4 + 8(j>>2),  l = t/8, j = t%8
// inside the tile (csrc/bindings.cpp:51-75).
//
// Work split used by every kernel here: one lane owns a "32-state group"
// q = 0..7 of a tile, i.e. the tile's values [32q, 32q+32).  Their windows end
// at bits 32Kq + (u+1)K, u = 0..31, so the group needs exactly the K words
// [Kq, Kq+K) plus the word before them (the tile's last word for q = 0).
// Those 32 values are columns q and q+8 of the tile, each with all 16 k rows:
//   run h = 0 (u = 0..15)  -> k in {0,1,8,9,2,3,10,11} + 0
//   run h = 1 (u = 16..31) -> k in {0,1,8,9,2,3,10,11} + 4
// for column q from u%16 in {0,1,2,3,8,9,10,11} and for column q+8 from
// u%16 in {4,5,6,7,12,13,14,15}.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <utility>

namespace exl3 {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr float kHadNorm = 0.08838834764831845f;  // 1/sqrt(128)

// Global-address-space view of a pointer.  Pointers read from tables or
// selected at run time are generic to the compiler, which then emits FLAT
// loads; those count against the LDS counter too, so every LDS wait would
// also wait for all outstanding HBM loads.  Global loads keep them apart.
#define EXL3_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ EXL3_GLOBAL T* gptr(T* p) {
    return (EXL3_GLOBAL T*)p;
}

// ------------------------------------------------------- cross-lane moves

// Value of v held by lane (lane ^ J) of the wave, J in {1, 2, 4, 8, 16, 32},
// with DPP moves and the gfx950 permlane swaps: plain VALU, no LDS round trip
// (the generic shuffle lowers to ds_bpermute).
template <int J>
__device__ __forceinline__ float lane_xor(float v) {
    const int iv = __float_as_int(v);
    int r;
    if constexpr (J == 1) {
        r = __builtin_amdgcn_mov_dpp(iv, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    } else if constexpr (J == 2) {
        r = __builtin_amdgcn_mov_dpp(iv, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    } else if constexpr (J == 4) {
        const int t = __builtin_amdgcn_mov_dpp(iv, 0x141, 0xF, 0xF, false);  // row_half_mirror: lane ^ 7
        r = __builtin_amdgcn_mov_dpp(t, 0x1B, 0xF, 0xF, false);              // quad_perm [3,2,1,0]: ^ 3
    } else if constexpr (J == 8) {
        r = __builtin_amdgcn_mov_dpp(iv, 0x128, 0xF, 0xF, false);  // row_ror:8
    } else if constexpr (J == 16) {
        // rows 2r / 2r+1 exchanged: the first result holds the even row in
        // both, the second the odd row in both
        const auto sw = __builtin_amdgcn_permlane16_swap(iv, iv, false, false);
        r = (threadIdx.x & 16) ? (int)sw[0] : (int)sw[1];
    } else {
        static_assert(J == 32, "lane_xor: J must be a power of two below 64");
        const auto sw = __builtin_amdgcn_permlane32_swap(iv, iv, false, false);
        r = (threadIdx.x & 32) ? (int)sw[0] : (int)sw[1];
    }
    return __int_as_float(r);
}

template <int J>
__device__ __forceinline__ void fwht_stage(float& a, float& b, int lane) {
    const float pa = lane_xor<J>(a), pb = lane_xor<J>(b);
    if (lane & J) {
        a = pa - a;
        b = pb - b;
    } else {
        a = a + pa;
        b = b + pb;
    }
}

// Unnormalised 128-point Walsh-Hadamard transform of one wave's 128 values,
// value 2*lane in a and 2*lane+1 in b.  Radix-2 stages of stride 1, 2, ..., 64
// in that order, each (x[i] + x[i+h], x[i] - x[i+h]): the same float
// operations in the same order as the reference's hadamard
// (csrc/exl3_dequant.cuh:137-148), so results are bit-identical.
__device__ __forceinline__ void fwht128_pair_f(float& a, float& b, int lane) {
    const float s = a + b, d = a - b;
    a = s;
    b = d;
    fwht_stage<1>(a, b, lane);
    fwht_stage<2>(a, b, lane);
    fwht_stage<4>(a, b, lane);
    fwht_stage<8>(a, b, lane);
    fwht_stage<16>(a, b, lane);
    fwht_stage<32>(a, b, lane);
}

// fp16 round-to-nearest of a value already rounded to fp32.  Without the empty
// asm the backend folds the multiply (or fma) that produced v into
// v_fma_mixlo/hi_f16, which rounds the exact result to fp16 once: on MI355X
// that gave another fp16 for ~6e-5 of products, where the reference rounds
// the fp32 product (fp32 multiply, then __float2half_rn).
__device__ __forceinline__ _Float16 f16_rn(float v) {
    asm("" : "+v"(v));
    return (_Float16)v;
}
__device__ __forceinline__ __half2 h2_rn(float a, float b) {
    asm("" : "+v"(a), "+v"(b));
    return __floats2half2_rn(a, b);
}

// SiLU in fp32, g * sigmoid(g) = g / (1 + e^-g) (the reference's SwiGLU:
// csrc/p2b_moe.cu:283-290, src/sglang_exl3/exl3.py:1199-1206), with e^-g as
// 2^(-g log2 e) and the quotient as g times a reciprocal, from the hardware's
// exp2 and reciprocal approximations (v_exp_f32, v_rcp_f32, about 1 ulp
// each): a few ulp of fp32 error, far below the fp16 rounding every caller
// applies, and 4 VALU ops instead of ~20 for a correctly rounded exp and
// divide (the wide-tile gate/up epilogue runs 64 of these per lane per tile).
// e^-g overflowing to inf gives 0 (g -> -inf), e^-g -> 0 gives g.
__device__ __forceinline__ float silu_f(float g) {
    return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.4426950408889634f));
}

// +1.0f where bit J of lane is clear, -1.0f where it is set.
template <int J>
__device__ __forceinline__ float lane_sign(int lane) {
    return __uint_as_float(0x3f800000u | ((uint32_t)(lane & J) << (31 - __builtin_ctz(J))));
}

// The same transform as fwht128_pair_f in about 20 VALU instead of ~50, with
// the same rounded magnitudes; a result that is exactly zero may differ in
// sign (fwht128_pair_f stays the path of the bit-exact operators).
//   * Stages of stride 2..16 (lane bits 0..3) run on values that carry the
//     sign s = (-1)^popcount(lane & done bits): each is one fma with the
//     partner's value as its DPP operand, h' = h + c p with c = -1 on the
//     upper lane, so h' = s (x + y) below and h' = -s (y - x) above (one
//     rounding of the same sum).  The partner always carries the same s.
//   * Strides 32 and 64 (lane bits 4, 5): a permlane16 / permlane32 swap of
//     (a, b) gives each lane both operands of a butterfly, which then runs in
//     registers; two more swaps restore value 2 lane in a and 2 lane + 1 in b.
//   * The final s is multiplied out (exact).
__device__ __forceinline__ void fwht128_pair_fast(float& a, float& b, int lane) {
    float x = a + b, y = a - b;
    const float c1 = lane_sign<1>(lane), c2 = lane_sign<2>(lane), c4 = lane_sign<4>(lane), c8 = lane_sign<8>(lane);
    float t, u;
    // The compiler does not fold a DPP move into v_fmac, so the four stages are
    // written out.  A VGPR written by a VALU op needs two wait states before a
    // DPP read of it: the s_nop count plus the VALU ops in between give them.
    asm(
        "s_nop 1\n\t"
        "v_fmac_f32_dpp %0, %0, %4 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %1, %1, %4 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 0\n\t"
        "v_fmac_f32_dpp %0, %0, %5 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %1, %1, %5 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 0\n\t"
        // lane ^ 4 = (lane ^ 7) ^ 3: row_half_mirror, then quad_perm [3,2,1,0]
        "v_mov_b32_dpp %2, %0 row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
        "v_mov_b32_dpp %3, %1 row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 0\n\t"
        "v_fmac_f32_dpp %0, %2, %6 quad_perm:[3,2,1,0] row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %1, %3, %6 quad_perm:[3,2,1,0] row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 0\n\t"
        "v_fmac_f32_dpp %0, %0, %7 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %1, %1, %7 row_ror:8 row_mask:0xf bank_mask:0xf"
        : "+v"(x), "+v"(y), "=&v"(t), "=&v"(u)
        : "v"(c1), "v"(c2), "v"(c4), "v"(c8));
    // rows (r0, r1, r2, r3): a' = (x.r0, y.r0, x.r2, y.r2), b' = (x.r1, y.r1, x.r3, y.r3)
    auto w = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(y), false, false);
    float p = __uint_as_float(w[0]), q = __uint_as_float(w[1]);
    x = p + q;
    y = p - q;
    // halves: a' = (x.lo, y.lo), b' = (x.hi, y.hi)
    w = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
    p = __uint_as_float(w[0]);
    q = __uint_as_float(w[1]);
    x = p + q;
    y = p - q;
    w = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
    w = __builtin_amdgcn_permlane16_swap(w[0], w[1], false, false);
    const float s = __uint_as_float(0x3f800000u | ((uint32_t)__builtin_popcount(lane & 15) << 31));
    a = __uint_as_float(w[0]) * s;
    b = __uint_as_float(w[1]) * s;
}

// The same transform with one row held as 16 consecutive values per lane over
// 8 lanes (value 16 (lane & 7) + e in v[e]): stages of stride 1 .. 8 in
// registers, 16 .. 64 across the lanes (xor 1, 2, 4), in the order of
// fwht128_pair_f and with the same rounded magnitudes; like fwht128_pair_fast,
// a result that is exactly zero may differ in sign.  The lane stages run on
// values that carry a sign, as in fwht128_pair_fast: lane L forms v + c p with
// the partner's value p as the DPP operand of one v_fmac (c = -1 where bit J
// of L is set), which is x + y on the lower lane and -(x - y) on the upper one.
// Both lanes of every later pair carry the same sign, so after the three
// stages lane L holds (-1)^popcount(L & 7) times the transform, and
// fwht_x16_norm(L) is that sign times 1/sqrt(128).  One asm block per stage:
// the compiler does not fold a DPP move into v_fmac, and a VGPR written by a
// VALU op needs two wait states before a DPP read of it (the leading s_nop;
// inside a block each register is read 16 instructions after it is written).
#define EXL3_R16(X) X(0) X(1) X(2) X(3) X(4) X(5) X(6) X(7) X(8) X(9) X(10) X(11) X(12) X(13) X(14) X(15)
#define EXL3_X16_V(i) [v##i] "+v"(v[i]),
#define EXL3_X16_T(i) [t##i] "=&v"(t[i]),
__device__ __forceinline__ void fwht128_x16(float (&v)[16], int lane) {
#pragma unroll
    for (int h = 1; h < 16; h <<= 1)
#pragma unroll
        for (int e = 0; e < 16; ++e)
            if (!(e & h)) {
                const float x = v[e], y = v[e | h];
                v[e] = x + y;
                v[e | h] = x - y;
            }
    // the signs are listed as in-out operands only to close the operand lists
    float c1 = lane_sign<1>(lane), c2 = lane_sign<2>(lane), c4 = lane_sign<4>(lane);
    asm("s_nop 1\n\t"
#define EXL3_X16_S(i) "v_fmac_f32_dpp %[v" #i "], %[v" #i "], %[c] quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
        EXL3_R16(EXL3_X16_S)
#undef EXL3_X16_S
        : EXL3_R16(EXL3_X16_V) [c] "+v"(c1));
    asm("s_nop 1\n\t"
#define EXL3_X16_S(i) "v_fmac_f32_dpp %[v" #i "], %[v" #i "], %[c] quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf\n\t"
        EXL3_R16(EXL3_X16_S)
#undef EXL3_X16_S
        : EXL3_R16(EXL3_X16_V) [c] "+v"(c2));
    // lane ^ 4 = (lane ^ 7) ^ 3: row_half_mirror, then quad_perm [3,2,1,0]
    float t[16];
    asm("s_nop 1\n\t"
#define EXL3_X16_M(i) "v_mov_b32_dpp %[t" #i "], %[v" #i "] row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
        EXL3_R16(EXL3_X16_M)
#undef EXL3_X16_M
#define EXL3_X16_S(i) "v_fmac_f32_dpp %[v" #i "], %[t" #i "], %[c] quad_perm:[3,2,1,0] row_mask:0xf bank_mask:0xf\n\t"
        EXL3_R16(EXL3_X16_S)
#undef EXL3_X16_S
        : EXL3_R16(EXL3_X16_V) EXL3_R16(EXL3_X16_T) [c] "+v"(c4));
}
#undef EXL3_X16_T
#undef EXL3_X16_V
#undef EXL3_R16

__device__ __forceinline__ float fwht_x16_norm(int lane) {
    return (__builtin_popcount(lane & 7) & 1) ? -kHadNorm : kHadNorm;
}

// Sum of v over the 64 lanes of the wave (every lane gets the same total,
// accumulated in a fixed order).
__device__ __forceinline__ float wave_sum(float v) {
    v += lane_xor<32>(v);
    v += lane_xor<16>(v);
    v += lane_xor<8>(v);
    v += lane_xor<4>(v);
    v += lane_xor<2>(v);
    v += lane_xor<1>(v);
    return v;
}

// k offsets (inside a 16-row tile) of the 8 values one run gives one column,
// in decode order; the second run adds 4.
__host__ __device__ constexpr int kofs(int e) {
    return e == 0 ? 0 : e == 1 ? 1 : e == 2 ? 8 : e == 3 ? 9 : e == 4 ? 2 : e == 5 ? 3 : e == 6 ? 10 : 11;
}

// ------------------------------------------------------------------ windows

// 16-bit window of local value u (0..31) from the lane's word buffer
// buf[0] = previous word, buf[1..K] = own words.  Shifts are compile-time.
template <int K, int U>
__device__ __forceinline__ uint32_t window(const uint32_t* buf) {
    constexpr int rel_end = 32 + (U + 1) * K;
    constexpr int rel_start = rel_end - 16;
    constexpr int ia = rel_start / 32;
    constexpr int ib = (rel_end - 1) / 32;
    constexpr int sh = 32 * (ib + 1) - rel_end;
    if constexpr (ia == ib) {
        return __builtin_amdgcn_ubfe(buf[ib], sh, 16);
    } else {
        return __builtin_amdgcn_alignbit(buf[ia], buf[ib], sh) & 0xffffu;
    }
}

// Same window, with the straddling ones cut from the "middle words"
// mid[j] = bits 16..47 of buf[j]:buf[j+1] (one v_alignbit per word boundary,
// shared by every window crossing it) by a single v_bfe each.
template <int K, int U>
__device__ __forceinline__ uint32_t window_mid(const uint32_t* buf, const uint32_t* mid) {
    constexpr int rel_end = 32 + (U + 1) * K;
    constexpr int rel_start = rel_end - 16;
    constexpr int ia = rel_start / 32;
    constexpr int ib = (rel_end - 1) / 32;
    constexpr int sh = 32 * (ib + 1) - rel_end;
    if constexpr (ia == ib) {
        return __builtin_amdgcn_ubfe(buf[ib], sh, 16);
    } else {
        static_assert(sh > 16 && sh < 32, "a straddling window starts inside the middle word");
        return __builtin_amdgcn_ubfe(mid[ia], sh - 16, 16);
    }
}

// ---------------------------------------------------------------- codebooks

// x = state * M (+ 64248484 for 3INST) mod 2^32: one v_mul_lo_u32 (a
// 4-cycle VALU op on gfx950, like v_bfe_u32; building the product from
// 16-bit pieces takes at least two such ops).
template <int CB>
__device__ __forceinline__ uint32_t hash(uint32_t s) {
    constexpr uint32_t M = CB == 0 ? 89226354u : CB == 1 ? 0xCBAC1FEDu : 0x83DCD12Du;
    uint32_t x = s * M;
    if constexpr (CB == 0) x += 64248484u;
    return x;
}

__device__ __forceinline__ uint32_t cb_mask(uint32_t x) { return (x & 0x8fff8fffu) ^ 0x3b603b60u; }

// Sum of the four bytes of x plus acc (the mul1 codebook's byte sum), as one
// v_sad_u8 (sum of |byte - 0|).  v_sad_u8 is a plain VALU op: the dot-product
// form (v_dot4_u32_u8) fed straight into an MFMA operand gave wrong products
// on gfx950 (its result was consumed by the MFMA one instruction later).
__device__ __forceinline__ uint32_t byte_sum(uint32_t x, uint32_t acc) { return __builtin_amdgcn_sad_u8(x, 0u, acc); }

// Round-to-nearest decode of two states into a packed half2 (the rounding of
// the reference's CUDA kernels, csrc/quant/codebook.cuh:41,53,65,74,88).
template <int CB>
__device__ __forceinline__ uint32_t decode2_rn(uint32_t s0, uint32_t s1) {
    uint32_t x0 = hash<CB>(s0), x1 = hash<CB>(s1);
    if constexpr (CB == 2) {
        uint32_t h0 = byte_sum(x0, 0x6400u);
        uint32_t h1 = byte_sum(x1, 0x6400u);
        uint32_t p = __builtin_amdgcn_perm(h1, h0, 0x05040100u);
        __half2 hp = *reinterpret_cast<__half2*>(&p);
        const __half2 kinv = __halves2half2(__ushort_as_half(0x1eee), __ushort_as_half(0x1eee));
        const __half2 bias = __halves2half2(__ushort_as_half(0xc931), __ushort_as_half(0xc931));
        __half2 r = __hfma2(hp, kinv, bias);
        return *reinterpret_cast<uint32_t*>(&r);
    } else {
        uint32_t y0 = cb_mask(x0), y1 = cb_mask(x1);
        __half2 a = *reinterpret_cast<__half2*>(&y0);
        __half2 b = *reinterpret_cast<__half2*>(&y1);
        __half v0 = __hadd(__low2half(a), __high2half(a));
        __half v1 = __hadd(__low2half(b), __high2half(b));
        __half2 r = __halves2half2(v0, v1);
        return *reinterpret_cast<uint32_t*>(&r);
    }
}

// Exact fp32 value of a codebook entry (every intermediate is exact).
template <int CB>
__device__ __forceinline__ float decode_exact(uint32_t s) {
    uint32_t x = hash<CB>(s);
    if constexpr (CB == 2) {
        uint32_t h = byte_sum(x, 0x6400u);
        // h * 0x1eee + 0xc931: 0x1eee = 1774 * 2^-18, 0xc931 = -2721792 * 2^-18;
        // the product and the sum are exact in fp32.
        float hf = __half2float(__ushort_as_half((unsigned short)h));
        return hf * (1774.0f / 262144.0f) + (-2721792.0f / 262144.0f);
    } else {
        uint32_t y = cb_mask(x);
        return __half2float(__ushort_as_half((unsigned short)(y & 0xffffu))) +
               __half2float(__ushort_as_half((unsigned short)(y >> 16)));
    }
}

// Truncating decode of two states (the reference's host dequant rounding,
// csrc/exl3_dequant.cuh:41-55): exact fp32 value, then fp16 round-toward-zero.
template <int CB>
__device__ __forceinline__ uint32_t decode2_rz(uint32_t s0, uint32_t s1) {
    float a = decode_exact<CB>(s0), b = decode_exact<CB>(s1);
    auto r = __builtin_amdgcn_cvt_pkrtz(a, b);
    return *reinterpret_cast<uint32_t*>(&r);
}

// ------------------------------------------------------------- group decode

// Matmul-side decode ("pair form"): one 32-bit word per value, holding two
// fp16 numbers whose contribution to the product is their sum times x:
//   3INST / MCG: the two masked halves (lo, hi) — value = lo + hi, exactly the
//                pre-rounding sum the codebook adds (codebook.cuh:56-75);
//   mul1:        (h, -1534) with h = 1024 + byte_sum — value = kinv*h + bias
//                = kinv*(h - 1534) + delta, so the product is accumulated on
//                (h - 1534) and scaled by kinv (+ delta * sum(x)) afterwards
//                (codebook.cuh:76-89).
// The matmul pairs each word with the activation duplicated in both halves, so
// no fp16 add / fma is spent per value and the MFMA accumulates exactly in fp32.
constexpr uint32_t kMul1PairBias = 0xE5FE6400u;  // high half: fp16(-1534); low half: 0x6400
constexpr float kMul1Kinv = 1774.0f / 262144.0f;  // fp16 0x1eee
// delta = bias + 1534 * kinv = (-2721792 + 1534 * 1774) * 2^-18
constexpr float kMul1Delta = (float)(-2721792 + 1534 * 1774) / 262144.0f;

template <int CB>
__device__ __forceinline__ uint32_t decode_pair_word(uint32_t s) {
    const uint32_t x = hash<CB>(s);
    if constexpr (CB == 2) return byte_sum(x, kMul1PairBias);
    else return cb_mask(x);
}

// Pair-form value order of a lane's group (the GEMV and MoE kernels decode
// u = 4F .. 4F + 3 per MFMA fragment F): writing u = 8Q + 4c + t (Q = 0..3,
// c = 0..1, t = 0..3), value u is column q + 8c of the tile at row
// k = 4(Q >> 1) + kofs(4(Q & 1) + t), so each run of four consecutive values
// is one MFMA B fragment (one column, 4 rows).

// Tile row of value slot t (0..3) of quarter Q (0..3).
__host__ __device__ constexpr int quarter_row(int Q, int t) { return 4 * (Q >> 1) + kofs(4 * (Q & 1) + t); }

// mul1 raw entries: two states as the fp16 numbers 1024 + byte sum (exact,
// bits 0x6400 + sum), two VALU ops (v_sad_u8, v_sad_hi_u8) after the hashes.
// The value is kMul1Kinv * raw + kMul1Bias, an affine map the caller applies
// to the product: sum_k x_k v_k = kMul1Kinv * sum_k x_k raw_k + kMul1Bias * sum_k x_k.
constexpr float kMul1Bias = -2721792.0f / 262144.0f;  // fp16 0xc931
__device__ __forceinline__ uint32_t mul1_raw_pair(uint32_t s0, uint32_t s1) {
    return __builtin_amdgcn_sad_hi_u8(hash<2>(s1), 0u, __builtin_amdgcn_sad_u8(hash<2>(s0), 0u, 0x64006400u));
}

// Exact-rounding decode (dequant / decode ops): fp16 bits of two values.
// RAW (mul1, round to nearest): the raw entries of mul1_raw_pair instead.
// Windows come from buf and the middle words mid (window_mid).
template <int K, int CB, bool RZ, int H, int C, int P, bool RAW = false>
__device__ __forceinline__ uint32_t frag_pair(const uint32_t* buf, const uint32_t* mid) {
    constexpr int e0 = 2 * P, e1 = 2 * P + 1;
    constexpr int u0 = 16 * H + (e0 & 3) + 8 * (e0 >> 2) + 4 * C;
    constexpr int u1 = 16 * H + (e1 & 3) + 8 * (e1 >> 2) + 4 * C;
    uint32_t s0 = window_mid<K, u0>(buf, mid), s1 = window_mid<K, u1>(buf, mid);
    if constexpr (RAW) {
        static_assert(CB == 2 && !RZ, "raw entries: mul1, matmul side");
        return mul1_raw_pair(s0, s1);
    } else if constexpr (RZ) {
        return decode2_rz<CB>(s0, s1);
    } else {
        return decode2_rn<CB>(s0, s1);
    }
}

template <int K, int CB, bool RZ, int H, int C, bool RAW = false>
__device__ __forceinline__ void frag_decode(const uint32_t* buf, const uint32_t* mid, uint32_t* f) {
    f[0] = frag_pair<K, CB, RZ, H, C, 0, RAW>(buf, mid);
    f[1] = frag_pair<K, CB, RZ, H, C, 1, RAW>(buf, mid);
    f[2] = frag_pair<K, CB, RZ, H, C, 2, RAW>(buf, mid);
    f[3] = frag_pair<K, CB, RZ, H, C, 3, RAW>(buf, mid);
}

// Decode the 32 values of one lane's group into fp16 words frag[c][h][p]
// (values 2p, 2p+1 of column q + 8c, run h; tile row 4h + kofs(e)).  The
// straddling windows are cut from one middle word per word boundary (a
// single v_bfe each instead of v_alignbit + mask: config 3 gate/up M = 16 /
// 128 30.3 / 81.6 -> 29.6 / 79.5 us, MoE prefill 2048 tokens 528.6 -> 515.7).
template <int K, int CB, bool RZ, bool RAW = false>
__device__ __forceinline__ void decode_group(const uint32_t* buf, uint32_t frag[2][2][4]) {
    uint32_t mid[K];
#pragma unroll
    for (int j = 0; j < K; ++j) mid[j] = __builtin_amdgcn_alignbit(buf[j], buf[j + 1], 16);
    frag_decode<K, CB, RZ, 0, 0, RAW>(buf, mid, frag[0][0]);
    frag_decode<K, CB, RZ, 1, 0, RAW>(buf, mid, frag[0][1]);
    frag_decode<K, CB, RZ, 0, 1, RAW>(buf, mid, frag[1][0]);
    frag_decode<K, CB, RZ, 1, 1, RAW>(buf, mid, frag[1][1]);
}

}  // namespace exl3
