// EXL3 GEMM for many rows (prefill, fat experts) on gfx950 MFMA.
//
//   out[m][n] = svh[n] * (H . (A . T)[m][128-block]) / sqrt(128)
//
// A (fp16 [M][k]) arrives rotated (x * suh, FWHT, / sqrt(128)); T is the
// decoded trellis.  Reference: csrc/exl3_fat_gemm.cu:65-195 (tile GEMM +
// per-row output FWHT, plain or routed-scatter output).
//
// A workgroup owns an MT-row x 128-column output tile (4 waves, 32 columns
// each) and a range of k.  Per step (4 k-slices) a wave decodes one 32-value
// group per lane into four MFMA B fragments of real fp16 values (round to
// nearest, as the reference's device decode) and multiplies them with every
// row block of the staged A: v_mfma_f32_16x16x32_f16 consumes 32 real k values
// (twice the pair-form GEMV's rate: this kernel is MFMA-bound, not HBM-bound).
// A is staged per chunk of CH steps in LDS in the decode's k order (per
// 16-slice the 32-bit words [0,4,1,5 | 2,6,3,7]), so the A fragment of run h
// is one 16-byte LDS read.  Weights stream with D steps in flight.  The
// epilogue stages the fp32 tile in LDS, applies the output FWHT, norm and svh
// per row, and stores (fp32 or fp16), or adds atomically (k-splits, routed
// scatter with per-row weights).
#pragma once

#include "exl3_common.h"
#include "exl3_decode.h"
#include "exl3_gemv_impl.h"

namespace exl3 {

constexpr int FAT_THREADS = 256;  // 4 waves x 32 output columns
constexpr int FAT_CH = 4;         // steps per staged A chunk (256 k)
constexpr int FAT_ROWB = FAT_CH * 4 * 2 * 16 + 16;  // bytes per staged A row (+16: bank spread)

struct FatParams {
    const __half* a;          // [M][k] rotated activations
    const uint32_t* trellis;  // [k/16][n/16][16K] as words
    const __half* svh;        // [n]
    float* out32;             // [rows_out][n] fp32 output, or
    __half* out16;            // [M][n] fp16 output (plain store only)
    const int64_t* token_idx;  // scatter: destination row per input row (null: row m)
    const __half* route_w;     // scatter: weight per input row (null: 1)
    int M, k, n;
    int ksteps;      // steps (4 k-slices) per k-split
    int accumulate;  // add atomically into out32 instead of storing
};

template <int K>
__host__ __device__ constexpr int fat_depth() {
    return K <= 4 ? 4 : 2;
}

inline size_t fat_smem_bytes(int mt) {
    const size_t a = (size_t)mt * FAT_ROWB;
    const size_t c = (size_t)mt * 128 * sizeof(float);
    return a > c ? a : c;
}

template <int K, int CB, int MT>
__global__ __launch_bounds__(FAT_THREADS) void fat_gemm_kernel(FatParams p) {
    constexpr int RB = MT / 16;
    constexpr int D = fat_depth<K>();
    static_assert(FAT_CH % D == 0, "the register slot of a step must be static inside a chunk");
    extern __shared__ __align__(16) unsigned char fat_smem[];

    const int bx = blockIdx.x, sidx = blockIdx.z;
    const int m0 = blockIdx.y * MT;
    const int rows = min(MT, p.M - m0);
    const int tid = threadIdx.x, cw = tid >> 6, lane = tid & 63;
    const int g = lane >> 4, i = lane & 15, q = i & 7;
    const int ntiles = p.n >> 4;
    const int nsteps = p.ksteps;
    const int kt0 = sidx * nsteps * 4;
    const int nt = bx * 8 + cw * 2 + (i >> 3);
    const EXL3_GLOBAL uint32_t* tb = gptr(p.trellis) + ((size_t)(kt0 + g) * ntiles + nt) * (8 * K) + K * q;
    const size_t step_stride = (size_t)4 * ntiles * (8 * K);
    const int prev_addr = ((lane & ~7) | ((lane + 7) & 7)) << 2;
    const __half2 svv = ld_h2(gptr(p.svh) + bx * 128 + 2 * lane);  // epilogue scale, requested early

    float4_t acc[RB][2];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        acc[rb][0] = float4_t{0.f, 0.f, 0.f, 0.f};
        acc[rb][1] = float4_t{0.f, 0.f, 0.f, 0.f};
    }

    uint32_t w[D][K];
#pragma unroll
    for (int d = 0; d < D; ++d)
        if (d < nsteps) load_words<K>(tb + (size_t)d * step_stride, w[d]);

    const EXL3_GLOBAL __half* ag = gptr(p.a);
    for (int c0 = 0; c0 < nsteps; c0 += FAT_CH) {
        // stage the chunk's A: rows x (FAT_CH * 4) slices of 16 k, permuted
        if (c0) __syncthreads();  // every wave is done with the previous chunk
        for (int u = tid; u < MT * FAT_CH * 4; u += FAT_THREADS) {
            const int row = u / (FAT_CH * 4), sl = u - row * (FAT_CH * 4);
            u32x4_t lo = {0u, 0u, 0u, 0u}, hi = {0u, 0u, 0u, 0u};
            if (row < rows && c0 * 4 + sl < nsteps * 4) {
                const EXL3_GLOBAL u32x4_t* src = reinterpret_cast<const EXL3_GLOBAL u32x4_t*>(
                    ag + (size_t)(m0 + row) * p.k + (size_t)(kt0 + c0 * 4 + sl) * 16);
                lo = src[0];
                hi = src[1];
            }
            u32x4_t* dst = reinterpret_cast<u32x4_t*>(fat_smem + (size_t)row * FAT_ROWB + sl * 32);
            dst[0] = u32x4_t{lo.x, hi.x, lo.y, hi.y};  // k pairs (0,1) (8,9) (2,3) (10,11)
            dst[1] = u32x4_t{lo.z, hi.z, lo.w, hi.w};  // k pairs (4,5) (12,13) (6,7) (14,15)
        }
        __syncthreads();

#pragma unroll
        for (int s = 0; s < FAT_CH; ++s) {
            const int step = c0 + s;
            if (step >= nsteps) break;
            const int d = step % D;
            uint32_t buf[K + 1];
#pragma unroll
            for (int j = 0; j < K; ++j) buf[1 + j] = w[d][j];
            buf[0] = (uint32_t)__builtin_amdgcn_ds_bpermute(prev_addr, (int)buf[K]);
            uint32_t frag[2][2][4];
            decode_group<K, CB, false>(buf, frag);
            if (step + D < nsteps) load_words<K>(tb + (size_t)(step + D) * step_stride, w[d]);
            const unsigned char* arow = fat_smem + (size_t)i * FAT_ROWB + (s * 4 + g) * 32;
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                if (rb * 16 >= rows) break;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const half8_t A = *reinterpret_cast<const half8_t*>(arow + (size_t)rb * 16 * FAT_ROWB + h * 16);
#pragma unroll
                    for (int c = 0; c < 2; ++c) {
                        const half8_t B = *reinterpret_cast<const half8_t*>(frag[c][h]);
                        acc[rb][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, acc[rb][c], 0, 0, 0);
                    }
                }
            }
        }
    }

    // epilogue: fp32 tile through LDS, then one row per wave
    __syncthreads();
    float* ct = reinterpret_cast<float*>(fat_smem);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = rb * 16 + 4 * g + r;
                const int col = cw * 32 + (i >> 3) * 16 + (i & 7) + 8 * c;
                if (row < rows) ct[row * 128 + col] = acc[rb][c][r];
            }
    __syncthreads();
    const float sva = __low2float(svv), svb = __high2float(svv);
    const int c0 = bx * 128 + 2 * lane;
    for (int row = cw; row < rows; row += FAT_THREADS / 64) {
        float va = ct[row * 128 + 2 * lane], vb = ct[row * 128 + 2 * lane + 1];
        fwht128_pair_f(va, vb, lane);
        va = (va * kHadNorm) * sva;
        vb = (vb * kHadNorm) * svb;
        const int src = m0 + row;
        if (p.out16) {
            st_h2(gptr(p.out16) + (size_t)src * p.n + c0, __floats2half2_rn(va, vb));
            continue;
        }
        size_t dst = (size_t)src;
        if (p.token_idx) dst = (size_t)gptr(p.token_idx)[src];
        if (p.route_w) {
            const float rw = __half2float(__ushort_as_half(gptr(reinterpret_cast<const uint16_t*>(p.route_w))[src]));
            va *= rw;
            vb *= rw;
        }
        float* o = p.out32 + dst * p.n + c0;
        if (p.accumulate) {
            atomicAdd(o, va);
            atomicAdd(o + 1, vb);
        } else {
            const float2 v2 = make_float2(va, vb);
            *reinterpret_cast<EXL3_GLOBAL unsigned long long*>(gptr(o)) = *reinterpret_cast<const unsigned long long*>(&v2);
        }
    }
}

// ------------------------------------------------------------ wide tiles
//
// MFMA-bound shapes (many rows).  A workgroup of 4 waves owns 128 rows x 256
// columns; each wave 64 columns (two 32-value decode groups per lane) times
// all 128 rows, so each staged A fragment feeds four MFMAs and each decoded
// weight 128 rows.  Two workgroups share a CU (<= 256 registers per lane), so
// one wave's decode (VALU) runs beside the other's MFMAs.
//
// A is staged one step (64 k) at a time into two LDS buffers by direct
// global->LDS loads (global_load_lds_dwordx4: lane l writes bytes
// [16l, 16l+16) of the instruction's 1 KB), in natural k order with the
// 16-byte chunk index XOR-swizzled by row (chunk ^ (row & 7) ^ ((row >> 3) & 1)),
// which keeps the fragment reads conflict-free for 8- and 16-lane LDS phases.
// Natural k order works because each lane decodes all 16 k values of its two
// columns: fragment word j of run h' is tile rows (8h' + 2j, 8h' + 2j + 1).
//
// Step s: stage A of step s+1 into the other buffer, decode step s, request
// the weights of step s+1 into the registers just decoded, run the step's 64
// MFMAs; one barrier per step (its vmcnt(0) lands both requests).
constexpr int FB_ROWS = 128;
constexpr int FB_COLS = 256;                  // 4 waves x 64 columns
constexpr int FB_THREADS = 256;
constexpr int FB_STEP_BYTES = FB_ROWS * 128;  // 128 rows x 64 k fp16
constexpr int FB_PASS_ROWS = 32;              // epilogue rows per LDS pass
constexpr int FB_CTS = FB_COLS + 4;           // epilogue row stride (floats)
constexpr int FAT_MT_WIDE = 0;                // plan value (rows per tile) selecting fat_big_kernel

constexpr size_t fat_big_smem_bytes() {
    constexpr size_t stage = 2 * (size_t)FB_STEP_BYTES;
    constexpr size_t tile = (size_t)FB_PASS_ROWS * FB_CTS * sizeof(float);
    return stage > tile ? stage : tile;
}

// fp16 pair of tile rows (4H + kofs(2P), +1) of column q + 8C (round to nearest).
template <int K, int CB, int H, int C, int P>
__device__ __forceinline__ uint32_t nat_pair(const uint32_t* buf, const uint32_t* mid) {
    constexpr int e0 = 2 * P, e1 = 2 * P + 1;
    constexpr int u0 = 16 * H + (e0 & 3) + 8 * (e0 >> 2) + 4 * C;
    constexpr int u1 = 16 * H + (e1 & 3) + 8 * (e1 >> 2) + 4 * C;
    return decode2_rn<CB>(window_mid<K, u0>(buf, mid), window_mid<K, u1>(buf, mid));
}

// f[h'][j] = tile rows (8h' + 2j, +1) of column q + 8C: run H = j >> 1, pair P = h' + 2 (j & 1).
template <int K, int CB, int C>
__device__ __forceinline__ void nat_column(const uint32_t* buf, const uint32_t* mid, uint32_t (&f)[2][4]) {
    f[0][0] = nat_pair<K, CB, 0, C, 0>(buf, mid);
    f[0][1] = nat_pair<K, CB, 0, C, 2>(buf, mid);
    f[0][2] = nat_pair<K, CB, 1, C, 0>(buf, mid);
    f[0][3] = nat_pair<K, CB, 1, C, 2>(buf, mid);
    f[1][0] = nat_pair<K, CB, 0, C, 1>(buf, mid);
    f[1][1] = nat_pair<K, CB, 0, C, 3>(buf, mid);
    f[1][2] = nat_pair<K, CB, 1, C, 1>(buf, mid);
    f[1][3] = nat_pair<K, CB, 1, C, 3>(buf, mid);
}

// Decode one 32-value group (words w[0..K-1], previous word from lane q - 1).
template <int K, int CB>
__device__ __forceinline__ void nat_group(const uint32_t (&w)[K], int prev_addr, uint32_t (&f)[2][2][4]) {
    uint32_t buf[K + 1], mid[K];
#pragma unroll
    for (int j = 0; j < K; ++j) buf[1 + j] = w[j];
    buf[0] = (uint32_t)__builtin_amdgcn_ds_bpermute(prev_addr, (int)buf[K]);
#pragma unroll
    for (int j = 0; j < K; ++j) mid[j] = __builtin_amdgcn_alignbit(buf[j], buf[j + 1], 16);
    nat_column<K, CB, 0>(buf, mid, f[0]);
    nat_column<K, CB, 1>(buf, mid, f[1]);
}

template <int K, int CB>
__global__ __launch_bounds__(FB_THREADS, 2) void fat_big_kernel(FatParams p) {
    constexpr int RB = FB_ROWS / 16;
    constexpr int LOADS = FB_STEP_BYTES / 1024 / (FB_THREADS / 64);  // 1 KB direct loads per wave per step
    static_assert(LOADS % 2 == 0, "the row-parity swizzle bit must be static per load");
    extern __shared__ __align__(16) unsigned char fat_smem[];

    const int bx = blockIdx.x, sidx = blockIdx.z;
    const int m0 = blockIdx.y * FB_ROWS;
    const int rows = min(FB_ROWS, p.M - m0);
    const int tid = threadIdx.x, cw = tid >> 6, lane = tid & 63;
    const int g = lane >> 4, i = lane & 15, q = i & 7;
    const int ntiles = p.n >> 4;
    const int nsteps = p.ksteps;  // even
    const int kt0 = sidx * nsteps * 4;
    const int nt0 = bx * (FB_COLS / 16) + cw * 4 + (i >> 3);  // group G adds 2G tiles
    const EXL3_GLOBAL uint32_t* tb = gptr(p.trellis) + ((size_t)(kt0 + g) * ntiles + nt0) * (8 * K) + K * q;
    const size_t step_stride = (size_t)4 * ntiles * (8 * K);
    const int prev_addr = ((lane & ~7) | ((lane + 7) & 7)) << 2;

    // direct-load sources: load j of this wave fills LDS rows 8J .. 8J+7
    // (J = cw*LOADS + j); lane l writes row 8J + (l >> 3), physical chunk l & 7,
    // which holds logical chunk (l & 7) ^ (l >> 3) ^ (J & 1).  Rows past M
    // repeat the last row (their results are never stored).
    const EXL3_GLOBAL char* abase =
        reinterpret_cast<const EXL3_GLOBAL char*>(gptr(p.a)) + ((size_t)m0 * p.k + (size_t)kt0 * 16) * 2;
    uint32_t aoff[LOADS];
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
        const int J = cw * LOADS + j;
        const int row = min(8 * J + (lane >> 3), rows - 1);
        const int c = (lane & 7) ^ (lane >> 3) ^ (j & 1);
        aoff[j] = (uint32_t)row * (uint32_t)p.k * 2u + 16u * (uint32_t)c;
    }
    auto stage_a = [&](int step, int bufi) {
        const EXL3_GLOBAL char* src = abase + (size_t)step * 128;
#pragma unroll
        for (int j = 0; j < LOADS; ++j)
            __builtin_amdgcn_global_load_lds(
                reinterpret_cast<const EXL3_GLOBAL void*>(src + aoff[j]),
                (__attribute__((address_space(3))) void*)(fat_smem + (size_t)bufi * FB_STEP_BYTES +
                                                          (size_t)(cw * LOADS + j) * 1024),
                16, 0, 0);
    };
    // fragment reads: row 16rb + i, logical chunk 2g + h'
    uint32_t rd_off[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) rd_off[h] = (uint32_t)i * 128u + 16u * (uint32_t)((2 * g + h) ^ (i & 7) ^ (i >> 3));

    float4_t acc[RB][2][2];  // [row block][group][column half]
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int G = 0; G < 2; ++G)
#pragma unroll
            for (int c = 0; c < 2; ++c) acc[rb][G][c] = float4_t{0.f, 0.f, 0.f, 0.f};

    uint32_t w[2][K];  // [group][word] of the current step
    auto load_step = [&](int step) {
        const EXL3_GLOBAL uint32_t* t = tb + (size_t)step * step_stride;
        load_words<K>(t, w[0]);
        load_words<K>(t + 16 * K, w[1]);
    };
    load_step(0);
    stage_a(0, 0);
    __syncthreads();

    // buffer SL = s & 1 holds step s's staged A; requests past the last step are
    // clamped to it (no branch inside the unrolled body)
    auto step_body = [&](int s, auto slot_c) {
        constexpr int SL = decltype(slot_c)::value;
        const int next = s + 1 < nsteps ? s + 1 : s;
        stage_a(next, SL ^ 1);
        uint32_t fr[2][2][2][4];  // [group][column half][h'][j]
        nat_group<K, CB>(w[0], prev_addr, fr[0]);
        nat_group<K, CB>(w[1], prev_addr, fr[1]);
        load_step(next);
        // keep the decode and the MFMA phase apart: mixing them raises register
        // pressure past the 256 of two waves per SIMD (spills for some K)
        __builtin_amdgcn_sched_barrier(0);
        const unsigned char* buf = fat_smem + (size_t)SL * FB_STEP_BYTES;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const half8_t A = *reinterpret_cast<const half8_t*>(buf + rd_off[h] + rb * 2048);
#pragma unroll
                for (int G = 0; G < 2; ++G)
#pragma unroll
                    for (int c = 0; c < 2; ++c)
                        acc[rb][G][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            A, *reinterpret_cast<const half8_t*>(fr[G][c][h]), acc[rb][G][c], 0, 0, 0);
            }
        }
        __syncthreads();
    };
    for (int s = 0; s < nsteps; s += 2) {
        step_body(s, std::integral_constant<int, 0>{});
        step_body(s + 1, std::integral_constant<int, 1>{});
    }

    // epilogue: passes of 32 rows through LDS; per (row, 128-block) one wave
    // applies the output FWHT, norm and svh.  Accumulator (rb, G, c, r) is
    // row 16rb + 4g + r, column 64cw + 32G + 16(i >> 3) + (i & 7) + 8c.
    float* ct = reinterpret_cast<float*>(fat_smem);
    constexpr int PRB = FB_PASS_ROWS / 16;
#pragma unroll
    for (int pass = 0; pass < RB / PRB; ++pass) {
        if (pass * FB_PASS_ROWS >= rows) break;
        if (pass) __syncthreads();
#pragma unroll
        for (int rr = 0; rr < PRB; ++rr)
#pragma unroll
            for (int G = 0; G < 2; ++G)
#pragma unroll
                for (int c = 0; c < 2; ++c)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int row = rr * 16 + 4 * g + r;
                        const int col = cw * 64 + G * 32 + (i >> 3) * 16 + (i & 7) + 8 * c;
                        ct[row * FB_CTS + col] = acc[pass * PRB + rr][G][c][r];
                    }
        __syncthreads();
        const int prow = min(FB_PASS_ROWS, rows - pass * FB_PASS_ROWS);
        for (int item = cw; item < prow * (FB_COLS / 128); item += FB_THREADS / 64) {
            const int row = item / (FB_COLS / 128), b = item - row * (FB_COLS / 128);
            const float2 v = *reinterpret_cast<const float2*>(ct + row * FB_CTS + b * 128 + 2 * lane);
            float va = v.x, vb = v.y;
            const int c0 = bx * FB_COLS + b * 128 + 2 * lane;
            const __half2 sv = ld_h2(gptr(p.svh) + c0);
            fwht128_pair_f(va, vb, lane);
            va = (va * kHadNorm) * __low2float(sv);
            vb = (vb * kHadNorm) * __high2float(sv);
            const int src = m0 + pass * FB_PASS_ROWS + row;
            if (p.out16) {
                st_h2(gptr(p.out16) + (size_t)src * p.n + c0, __floats2half2_rn(va, vb));
                continue;
            }
            size_t dst = (size_t)src;
            if (p.token_idx) dst = (size_t)gptr(p.token_idx)[src];
            if (p.route_w) {
                const float rw =
                    __half2float(__ushort_as_half(gptr(reinterpret_cast<const uint16_t*>(p.route_w))[src]));
                va *= rw;
                vb *= rw;
            }
            float* o = p.out32 + dst * p.n + c0;
            if (p.accumulate) {
                atomicAdd(o, va);
                atomicAdd(o + 1, vb);
            } else {
                const float2 v2 = make_float2(va, vb);
                *reinterpret_cast<EXL3_GLOBAL unsigned long long*>(gptr(o)) =
                    *reinterpret_cast<const unsigned long long*>(&v2);
            }
        }
    }
}

template <int K>
int fat_launch_k(int cb, int mt, const FatParams& p, int splits, hipStream_t st) {
    if (mt == FAT_MT_WIDE) {
        dim3 grid(p.n / FB_COLS, (p.M + FB_ROWS - 1) / FB_ROWS, splits);
        const size_t smem = fat_big_smem_bytes();
#define EXL3_FATB(CBV)                                                                                 \
    if (cb == CBV) {                                                                                   \
        const void* fn = reinterpret_cast<const void*>(&fat_big_kernel<K, CBV>);                       \
        const int lrc = allow_dynamic_lds(fn, smem, "exl3 fat gemm (wide tiles)");                     \
        if (lrc) return lrc;                                                                           \
        fat_big_kernel<K, CBV><<<grid, FB_THREADS, smem, st>>>(p);                                     \
        return launch_status("exl3 fat gemm launch");                                                  \
    }
        EXL3_FATB(0) EXL3_FATB(1) EXL3_FATB(2)
#undef EXL3_FATB
    }
    dim3 grid(p.n / 128, (p.M + mt - 1) / mt, splits);
    const size_t smem = fat_smem_bytes(mt);
#define EXL3_FAT(CBV, MTV)                                                                             \
    if (cb == CBV && mt == MTV) {                                                                      \
        const void* fn = reinterpret_cast<const void*>(&fat_gemm_kernel<K, CBV, MTV>);                 \
        const int lrc = allow_dynamic_lds(fn, smem, "exl3 fat gemm");                                  \
        if (lrc) return lrc;                                                                           \
        fat_gemm_kernel<K, CBV, MTV><<<grid, FAT_THREADS, smem, st>>>(p);                              \
        return launch_status("exl3 fat gemm launch");                                                  \
    }
#define EXL3_FAT_CB(CBV) EXL3_FAT(CBV, 16) EXL3_FAT(CBV, 64) EXL3_FAT(CBV, 128)
    EXL3_FAT_CB(0) EXL3_FAT_CB(1) EXL3_FAT_CB(2)
#undef EXL3_FAT_CB
#undef EXL3_FAT
    set_error("exl3 fat gemm: no kernel for codebook %d tile rows %d", cb, mt);
    return EXL3_ERR_UNSUPPORTED;
}

// One instantiation unit per K (exl3_fat_inst.hip built with -DEXL3_K=K).
int fat_launch(int K, int cb, int mt, const FatParams& p, int splits, hipStream_t st);

}  // namespace exl3
