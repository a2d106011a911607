// Balanced EXL3 GEMV for up to 4 rows (bs <= 4) on gfx950:
// y = svh (.) H(x' . T) / sqrt(128).
//
// Same product as gemv_kernel (reference: csrc/quant/exl3_gemv_kernel.cuh:138-402),
// organised for an even load on every SIMD and a one-round-trip k reduction:
//
//   * Each 128-column block's k range (k/64 "k-steps" of 64) is cut into P
//     equal pieces; workgroup (pi, cb) (4 waves, one per 32 columns)
//     computes piece pi of block cb.  The planner picks P so that the
//     blocks x P workgroups spread evenly over the CUs.
//   * Each workgroup rotates only the activation blocks its piece needs, of
//     every row (x * suh, FWHT, / sqrt(128), fp16), into LDS in MFMA
//     A-fragment order; row r is A row r (lanes i = r read it).
//   * The decode/MFMA loop is gemv_kernel's (pair-form words, activations
//     duplicated), with four independent accumulator chains.
//   * Epilogue: the four waves' column slices meet in LDS, one wave per row
//     applies the output FWHT, 1/sqrt(128) and svh, and adds the result into
//     a 64-bit fixed-point accumulator per output element (atomic add with
//     return).  The accumulator's top bits count the contributions; the
//     workgroup whose add brings the count to P converts the sum to fp16,
//     stores y and clears the accumulator for the next call.  Integer
//     addition is associative, so the result does not depend on the order in
//     which workgroups arrive.
#pragma once

#include "exl3_gemv_impl.h"

namespace exl3 {

constexpr int SK_THREADS = 256;
#ifndef EXL3_SK_DEPTH_WORDS
#define EXL3_SK_DEPTH_WORDS 8
#endif

struct GemvSkParams {
    const __half* x;          // [m][k]
    const uint32_t* trellis;  // [k/16][n/16][8K] words
    const __half* suh;        // [k]
    const __half* svh;        // [n]
    __half* y;                // [m][n]
    unsigned long long* acc;  // [m][n] fixed-point accumulators, zero between calls
    int m, k, n;
    int pieces;  // P: workgroups per column block (grid.x); grid.y = n / 128
};

// Rows the kernel is instantiated for (MR >= m): 1, 2 or 4.
inline int gemv_sk_rows(int m) { return m <= 1 ? 1 : m <= 2 ? 2 : 4; }

inline size_t gemv_sk_smem_bytes(int ns, int mr) {
    // A staging [MR][NS * 4 k-tiles][4 quarters][8 halves] + zero fragment, x'
    // sums per row and step (mul1), one 128-column fp32 tile per row
    return (((size_t)mr * ns * 128 * 2 + 16 + 15) & ~(size_t)15) + (((size_t)mr * ns * 4 + 15) & ~(size_t)15) +
           (size_t)mr * 128 * 4;
}

// One MFMA B fragment (values u = 4F..4F+3 of the lane's group, pair form)
// multiplied into its accumulator chain (quarter parity x column tile) right
// after it is decoded; the middle words mid[] serve the straddling windows.
template <int K, int CB, int F>
__device__ __forceinline__ void sk_frag(const uint32_t* buf, const uint32_t* mid, const half8_t (&A)[4],
                                        float4_t (&acc)[2][2]) {
    uint32_t vf[4];
    vf[0] = decode_pair_word<CB>(window_mid<K, 4 * F + 0>(buf, mid));
    vf[1] = decode_pair_word<CB>(window_mid<K, 4 * F + 1>(buf, mid));
    vf[2] = decode_pair_word<CB>(window_mid<K, 4 * F + 2>(buf, mid));
    vf[3] = decode_pair_word<CB>(window_mid<K, 4 * F + 3>(buf, mid));
    const half8_t B = *reinterpret_cast<const half8_t*>(vf);
    constexpr int Q = F >> 1, c = F & 1;
    acc[Q & 1][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[Q], B, acc[Q & 1][c], 0, 0, 0);
}

template <int K, int CB, int... Fs>
__device__ __forceinline__ void sk_frags(const uint32_t* buf, const uint32_t* mid, const half8_t (&A)[4],
                                         float4_t (&acc)[2][2], std::integer_sequence<int, Fs...>) {
    (sk_frag<K, CB, Fs>(buf, mid, A, acc), ...);
}

// Weight steps in flight per wave: the whole piece when its words fit
// EXL3_SK_DEPTH_WORDS registers per lane, else two.
template <int K, int NS>
__host__ __device__ constexpr int sk_depth() {
    return NS * K <= EXL3_SK_DEPTH_WORDS ? NS : (gv_depth<K>() < NS ? gv_depth<K>() : NS);
}

template <int K, int CB, int NS, int MR>
__global__ __launch_bounds__(SK_THREADS) void gemv_sk_kernel(GemvSkParams p) {
    constexpr int D = sk_depth<K, NS>();
    extern __shared__ __align__(16) unsigned char sk_smem[];

    const int n = p.n, P = p.pieces, m = p.m, k = p.k;
    const int pi = blockIdx.x, cb = blockIdx.y;
    const int ks0 = pi * NS;  // first k-step of the piece

    const int tid = threadIdx.x, cw = tid >> 6, lane = tid & 63;
    const int g = lane >> 4, i = lane & 15, q = i & 7;
    const int ntiles = n >> 4;

    constexpr int ROWH = NS * 128;  // staged halves per row
    _Float16* xs = reinterpret_cast<_Float16*>(sk_smem);
    float* xsum = reinterpret_cast<float*>(sk_smem + (((size_t)MR * ROWH * 2 + 16 + 15) & ~(size_t)15));
    float* ybuf = xsum + ((MR * NS + 3) & ~3);

    // rotation work: the 128-blocks j0..j0+nblocks-1 holding the piece's
    // k-steps, for each row: jobs = m * nblocks, wave cw takes jobs cw, cw + 4, ..
    const int j0 = ks0 >> 1;
    const int nblocks = ((ks0 + NS - 1) >> 1) - j0 + 1;
    const int jobs = m * nblocks;

    // 1. activations of this wave's first job, then the weights
    const EXL3_GLOBAL __half* xg = gptr(p.x) + 2 * lane;
    const EXL3_GLOBAL __half* suhg = gptr(p.suh) + 2 * lane;
    __half2 x0 = __float2half2_rn(0.f), s0 = x0;
    if (cw < jobs) {
        const int r0 = cw / nblocks, b0 = cw - r0 * nblocks;
        x0 = ld_h2(xg + (size_t)r0 * k + (j0 + b0) * 128);
        s0 = ld_h2(suhg + (j0 + b0) * 128);
    }
    const int nt = cb * 8 + cw * 2 + (i >> 3);
    const size_t ss = (size_t)4 * ntiles * (8 * K);  // words between k-steps
    const EXL3_GLOBAL uint32_t* tb = gptr(p.trellis) + ((size_t)(ks0 * 4 + g) * ntiles + nt) * (8 * K) + K * q;
    const __half2 svv = ld_h2(gptr(p.svh) + cb * 128 + 2 * lane);
    // only the first step's words now; the rest of the ring after the
    // staging barrier, so that the burst every wave issues at its start is
    // one step (7.3 MB over the grid at config 2, not 14.7) and the decode
    // starts sooner (config 2 m = 1: 10.64 -> 10.43 us)
    uint32_t w[D][K];
    load_words<K>(tb, w[0]);

    // 2. input rotation into LDS (A order, each value duplicated).  A lane
    //    holds k = 128 j + 2 lane (+1): k-step 2j + lane/32, offset (2 lane) % 64
    //    inside it, so its LDS slot is a per-lane constant plus 128 halves per
    //    local step.
    if (tid < 8) xs[MR * ROWH + tid] = (_Float16)0.0f;
    // xs_index((2 lane) % 64, 0, 4 NS) in closed form: k-tile (lane / 8) % 4,
    // quarter lane % 4, value pair (lane / 4) % 2
    const int xs_lane = ((lane >> 3) & 3) * 32 + (lane & 3) * 8 + ((lane >> 2) & 1) * 4;
    for (int jb = cw; jb < jobs; jb += 4) {
        const int row = jb / nblocks, j = j0 + jb - row * nblocks;
        const int l = 2 * j + (lane >> 5) - ks0;  // local step of this lane's values
        const bool mine = l >= 0 && l < NS;
        const __half2 xv = jb == cw ? x0 : ld_h2(xg + (size_t)row * k + j * 128);
        const __half2 sv = jb == cw ? s0 : ld_h2(suhg + j * 128);
        const __half2 pr = __hmul2(xv, sv);
        float a = __low2float(pr), c = __high2float(pr);
        fwht128_pair_fast(a, c, lane);
        const _Float16 ha = f16_rn(a * kHadNorm), hc = f16_rn(c * kHadNorm);
        if (mine) {
            // (ha, ha, hc, hc): the two values, each duplicated, in one 8-byte store
            const uint32_t da = (uint32_t)__builtin_bit_cast(unsigned short, ha) * 0x10001u;
            const uint32_t dc = (uint32_t)__builtin_bit_cast(unsigned short, hc) * 0x10001u;
            *reinterpret_cast<uint2*>(xs + row * ROWH + xs_lane + l * 128) = make_uint2(da, dc);
        }
        if constexpr (CB == 2) {
            // per-step sums over each half of the wave (lanes 0-31: k-step 2j, 32-63: 2j+1)
            float t = mine ? (float)ha + (float)hc : 0.f;
            t += lane_xor<16>(t);
            t += lane_xor<8>(t);
            t += lane_xor<4>(t);
            t += lane_xor<2>(t);
            t += lane_xor<1>(t);
            if ((lane & 31) == 0 && mine) xsum[row * NS + l] = t;
        }
    }
    __syncthreads();
#pragma unroll
    for (int d = 1; d < D; ++d) load_words<K>(tb + (size_t)(d < NS ? d : NS - 1) * ss, w[d]);

    // 3. decode + MFMA; four accumulator chains (quarter parity x column tile).
    //    Activation row r is A row r: lanes with i = r < m read it, the
    //    others keep zero fragments.
    float4_t acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a) {
        acc[a][0] = float4_t{0.f, 0.f, 0.f, 0.f};
        acc[a][1] = float4_t{0.f, 0.f, 0.f, 0.f};
    }
    const bool a_live = i < m;
    const _Float16* a_base = xs + (a_live ? i : 0) * ROWH + g * 32;
    const int prev_addr = ((lane & ~7) | ((lane + 7) & 7)) << 2;  // lane of group q - 1 (mod 8)
    half8_t A[4];
#pragma unroll
    for (int Q = 0; Q < 4; ++Q) A[Q] = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        const int d = s % D;
        uint32_t buf[K + 1];
#pragma unroll
        for (int j = 0; j < K; ++j) buf[1 + j] = w[d][j];
        // the word before the group's first word: the previous group's last
        // word (group 0: the tile's last word, the bitstream is tail-biting)
        buf[0] = (uint32_t)__builtin_amdgcn_ds_bpermute(prev_addr, (int)buf[K]);
        if (a_live) {
#pragma unroll
            for (int Q = 0; Q < 4; ++Q) A[Q] = *reinterpret_cast<const half8_t*>(a_base + (s * 16 + Q) * 8);
        }
        uint32_t mid[K];
#pragma unroll
        for (int j = 0; j < K; ++j) mid[j] = __builtin_amdgcn_alignbit(buf[j], buf[j + 1], 16);
        // decode fragment by fragment, each MFMA issued as soon as its
        // fragment is ready so the matrix core runs under the next decode
        sk_frags<K, CB>(buf, mid, A, acc, std::make_integer_sequence<int, 8>{});
        if (s + D < NS) load_words<K>(tb + (size_t)(s + D) * ss, w[d]);
#pragma unroll
        for (int f = 0; f < 8; ++f) {
            __builtin_amdgcn_sched_group_barrier(0x002, 12, 0);  // VALU
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
        }
    }
    // output row r < 4 sits in lanes with g = 0, element r: column
    // cw*32 + (i >> 3)*16 + (i & 7) + 8c
    if (g == 0) {
        const int col = cw * 32 + (i >> 3) * 16 + (i & 7);
#pragma unroll
        for (int r = 0; r < MR; ++r)
            if (r < m) {
                ybuf[r * 128 + col] = acc[0][0][r] + acc[1][0][r];
                ybuf[r * 128 + col + 8] = acc[0][1][r] + acc[1][1][r];
            }
    }
    __syncthreads();
    if (cw >= m) return;
    const int r = cw;  // one output row per wave

    // 4. output FWHT, scale, fixed-point accumulate; the workgroup completing
    //    an element writes fp16 and clears its accumulator
    float a = ybuf[r * 128 + 2 * lane], b = ybuf[r * 128 + 2 * lane + 1];
    if constexpr (CB == 2) {
        float sx = 0.f;
#pragma unroll
        for (int l = 0; l < NS; ++l) sx += xsum[r * NS + l];
        a = a * kMul1Kinv + kMul1Delta * sx;
        b = b * kMul1Kinv + kMul1Delta * sx;
    }
    fwht128_pair_fast(a, b, lane);
    a = a * kHadNorm * __low2float(svv);
    b = b * kHadNorm * __high2float(svv);
    const size_t e0 = (size_t)r * n + cb * 128 + 2 * lane;
    fx_add_pair(p.acc + e0, a, b, P, gptr(p.y) + e0);
}

// Piece lengths (k-steps) the kernel is instantiated for.
constexpr int kSkSteps[] = {1, 2, 3, 4, 5, 6, 7, 8, 10, 12, 14, 16};

template <int K>
int gemv_sk_launch_k(int cb, int ns, const GemvSkParams& p, hipStream_t st) {
    const int mr = gemv_sk_rows(p.m);
    const size_t smem = gemv_sk_smem_bytes(ns, mr);
#define EXL3_SK_MR(CBV, NSV, MRV)                                                                      \
    if (cb == CBV && ns == NSV && mr == MRV) {                                                         \
        const void* fn = reinterpret_cast<const void*>(&gemv_sk_kernel<K, CBV, NSV, MRV>);             \
        const int lrc = allow_dynamic_lds(fn, smem, "exl3 gemv");                                      \
        if (lrc) return lrc;                                                                           \
        gemv_sk_kernel<K, CBV, NSV, MRV><<<dim3(p.pieces, p.n / 128), SK_THREADS, smem, st>>>(p);     \
        return launch_status("exl3 gemv launch");                                                      \
    }
#define EXL3_SK(CBV, NSV) EXL3_SK_MR(CBV, NSV, 1) EXL3_SK_MR(CBV, NSV, 2) EXL3_SK_MR(CBV, NSV, 4)
#define EXL3_SK_CB(CBV)                                                                                \
    EXL3_SK(CBV, 1) EXL3_SK(CBV, 2) EXL3_SK(CBV, 3) EXL3_SK(CBV, 4) EXL3_SK(CBV, 5) EXL3_SK(CBV, 6) EXL3_SK(CBV, 7)    \
    EXL3_SK(CBV, 8) EXL3_SK(CBV, 10) EXL3_SK(CBV, 12) EXL3_SK(CBV, 14) EXL3_SK(CBV, 16)
    EXL3_SK_CB(0) EXL3_SK_CB(1) EXL3_SK_CB(2)
#undef EXL3_SK_CB
#undef EXL3_SK
#undef EXL3_SK_MR
    set_error("exl3 gemv: no balanced kernel for codebook %d steps %d rows %d", cb, ns, p.m);
    return EXL3_ERR_UNSUPPORTED;
}

}  // namespace exl3
