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

// Wave priority 1 over the MFMA phase of the wide-tile kernel, so the matrix
// core is fed first while the SIMD's other wave decodes (config 3, M=2048:
// 552 -> 545 us before the ping-pong schedule; with it, priority 0 or raising
// the decoding wave instead measured 537 / 535 against 528 us).  Build with
// -DEXL3_FAT_SETPRIO=0 to leave priorities alone.
#ifndef EXL3_FAT_SETPRIO
#define EXL3_FAT_SETPRIO 1
#endif

constexpr int FAT_THREADS = 256;  // 4 waves x 32 output columns
constexpr int FAT_CH = 4;         // steps per staged A chunk (256 k)
constexpr int FAT_ROWB = FAT_CH * 4 * 2 * 16 + 16;  // bytes per staged A row (+16: bank spread)
// 16-row tiles stage 16 steps per chunk (33 KB of LDS: a 16-step k-split
// stages its whole A range once, with no barrier and reload in the middle of
// its steps; LDS then holds a CU to 4 workgroups): config 3 gate/up M = 16,
// kernel alone, graph-timed, 4 / 8 / 16 steps per chunk: 29.3 / 28.6 us (op)
// and 26.7 -> 26.1 us (kernel, 8 -> 16).  A partial last chunk is fine: its
// missing slices stage zeros and its steps are skipped.
template <int MT> __host__ __device__ constexpr int fat_ch() { return MT == 16 ? 16 : FAT_CH; }
template <int MT> __host__ __device__ constexpr int fat_rowb() { return fat_ch<MT>() * 4 * 2 * 16 + 16; }

// A run of rows of one expert in compact (expert-sorted) order: one row tile
// of the grouped mode, written by the MoE prefill routing kernel.
struct alignas(16) FatTile {
    int e;      // expert id
    int crow0;  // first compact row
    int nrows;  // 1..MT
    int pad;
};

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
    // Gate/up mode (fat_big_kernel<.., GU = true>): `trellis`/`svh` are the
    // gate projection, `trellis2`/`svh2` the up projection, both n wide;
    // out16[m][n] = fp16( silu(min(g, limit)) * clamp(u, -limit, limit) ).
    // fat_gemm_kernel in gate/up mode: grid.x enumerates (column block,
    // projection) pairs (even: gate, odd: up); each workgroup stores its fp32
    // partial tile, and the last of the 2 S arrivals of a (column block, row
    // tile) sums them, applies both output rotations and the SwiGLU.
    int gu;
    // Narrow split hand-off (gate/up mode, or plain mode with handoff) with
    // split_out != 0: each workgroup stores its partial tile and exits (no
    // counter, no last arrival); the launch of fat_split_finish_kernel that
    // follows sums and finishes every row.
    int split_out;
    const uint32_t* trellis2;
    const __half* svh2;
    float limit;  // <= 0 or inf: no clamp
    float* partials;  // [n/128][2][S][M][128] (narrow gate/up mode), [n/128][S][M][128] (handoff)
    int* counters;    // [n/128][row tiles], zero between calls
    // fat_gemm_kernel plain mode with k-splits and fp16 output (handoff != 0):
    // the same partial-tile hand-off with one projection; the last of the S
    // arrivals of a (column block, row tile) applies the epilogue and stores
    // out16 (deterministic, no fp32 atomics, zero fill or conversion pass).
    int handoff;
    // Grouped mode of fat_gemm_kernel (MoE prefill), gmode != 0: blockIdx.y
    // indexes `tiles` (tiles at or past *ntiles exit at once, so the grid is
    // static), `a` holds the rows in compact order, and the weights are the
    // tile's expert's entries of the nine per-expert tables (gate, up, down x
    // trellis, suh, svh).  One k-split.
    //   gmode 1 (gate): g32[crow][n] = fp32 gate output;
    //   gmode 2 (up):   out16[crow][n] = fp16(H(fp16(silu(min(g, L)) * clamp(u, -L, L)) (.) suh_down) / sqrt(128)),
    //                   the activation already rotated for the down projection;
    //   gmode 3 (down): out16[rows_map[crow]][n] = fp16 down output, by (token, slot) entry.
    int gmode;
    const FatTile* tiles;
    const int* ntiles;
    const int64_t* tabs[9];
    float* g32;
    const int* rows_map;
    // Tail split of the wide-tile kernel (one k-split, plain stores; 1-D grid
    // when tail_tiles > 0): tiles [0, tail_first) run whole, each of the
    // tail_tiles tiles after them as two k-halves (workgroups tail_first + 2j
    // and + 1 for tile tail_first + j), so a last round of workgroups that
    // would leave at least half the CUs idle fills them.  The first half to
    // finish stores its accumulators device-coherently in tail_part and
    // raises a flag; the second adds them to its own and runs the epilogue.
    int tail_first, tail_tiles, tiles_x;
    float* tail_part;  // [tail_tiles][FB_TAIL_FLOATS]
    int* tail_sync;    // [tail_tiles] arrival counts, then [tail_tiles] flags; zero between calls
    int max_polls;     // polls before the second half's wait gives up
    int* status;       // workspace status word: EXL3_WAIT_FAT_TAIL when a wait gave up
    // Narrow kernel on mul1 weights (fat_gemm_kernel<.., RAW = true>, plain
    // and gate/up modes): B holds the raw entries (mul1_raw_pair) and the
    // epilogue applies kMul1Kinv * acc + kMul1Bias * (sum of the rows' x over
    // the k range), from rowsum[row][k/128] (rotate_rows_kernel's chunk sums).
    const float* rowsum;
};

// Sum over chunks [c0, c0 + nc) of row `row` of rowsum (one wave).
__device__ __forceinline__ float fat_row_sum(const float* rowsum, int nchk, int row, int c0, int nc, int lane) {
    const float* r = rowsum + (size_t)row * nchk + c0;
    float v = 0.f;
    for (int c = lane; c < nc; c += 64) v += gptr(r)[c];
    return wave_sum(v);
}

template <int K>
__host__ __device__ constexpr int fat_depth() {
    return K <= 4 ? 4 : 2;
}

inline size_t fat_smem_bytes(int mt) {
    const size_t a = (size_t)mt * (mt == 16 ? fat_rowb<16>() : FAT_ROWB);
    const size_t c = (size_t)mt * 128 * sizeof(float);
    return a > c ? a : c;
}

// Gate/up epilogue of one output row segment (two columns per lane of a
// 128-column block): the summed gate and up partials -> (mul1 map: times
// kMul1Kinv plus sx, the row's bias term) -> both output rotations, svh ->
// clamp -> fp16(silu(g) * u) at out16[orow][c0].
template <bool RAW>
__device__ __forceinline__ void fat_gu_finish(const FatParams& p, size_t orow, int c0, float ga, float gb, float ua,
                                              float ub, float sx, __half2 svg, __half2 svu, int lane) {
    if constexpr (RAW) {
        ga = ga * kMul1Kinv + sx;
        gb = gb * kMul1Kinv + sx;
        ua = ua * kMul1Kinv + sx;
        ub = ub * kMul1Kinv + sx;
    }
    fwht128_pair_fast(ga, gb, lane);
    fwht128_pair_fast(ua, ub, lane);
    ga = (ga * kHadNorm) * __low2float(svg);
    gb = (gb * kHadNorm) * __high2float(svg);
    ua = (ua * kHadNorm) * __low2float(svu);
    ub = (ub * kHadNorm) * __high2float(svu);
    if (p.limit > 0.0f && p.limit < __builtin_huge_valf()) {
        ga = fminf(ga, p.limit);
        gb = fminf(gb, p.limit);
        ua = fminf(fmaxf(ua, -p.limit), p.limit);
        ub = fminf(fmaxf(ub, -p.limit), p.limit);
    }
    st_h2(gptr(p.out16) + orow * p.n + c0, h2_rn(silu_f(ga) * ua, silu_f(gb) * ub));
}

// At least four waves per SIMD for 16- and 64-row tiles (75-80 / 90 VGPRs at
// K = 3, no spills: 6 / 5 waves; 64-row tiles are held to 4 by their LDS).
template <int K, int CB, int MT, bool RAW = false>
__global__ __launch_bounds__(FAT_THREADS, MT <= 64 ? 4 : 1) void fat_gemm_kernel(FatParams p) {
    static_assert(!RAW || CB == 2, "raw entries: mul1");
    constexpr int RB = MT / 16;
    constexpr int D = fat_depth<K>();
    constexpr int CH = fat_ch<MT>(), ROWB = fat_rowb<MT>();
    static_assert(CH % D == 0, "the register slot of a step must be static inside a chunk");
    extern __shared__ __align__(16) unsigned char fat_smem[];

    const int sidx = blockIdx.z;
    // gate/up mode: blockIdx.x = 2 * column block + projection
    const int bx = p.gu ? (int)(blockIdx.x >> 1) : (int)blockIdx.x;
    const uint32_t* trel = (p.gu && (blockIdx.x & 1)) ? p.trellis2 : p.trellis;
    const __half* svh_p = p.svh;
    const __half* dsuh = nullptr;  // grouped up pass: the down projection's suh
    int m0 = blockIdx.y * MT;
    int rows = min(MT, p.M - m0);
    if (p.gmode) {
        if ((int)blockIdx.y >= __builtin_amdgcn_readfirstlane(*gptr(p.ntiles))) return;
        const EXL3_GLOBAL FatTile* tl = gptr(p.tiles) + blockIdx.y;
        const int e = __builtin_amdgcn_readfirstlane(tl->e);
        m0 = __builtin_amdgcn_readfirstlane(tl->crow0);
        rows = __builtin_amdgcn_readfirstlane(tl->nrows);
        const int pb = p.gmode == 1 ? 0 : (p.gmode == 2 ? 3 : 6);
        trel = reinterpret_cast<const uint32_t*>(gptr(p.tabs[pb])[e]);
        svh_p = reinterpret_cast<const __half*>(gptr(p.tabs[pb + 2])[e]);
        if (p.gmode == 2) dsuh = reinterpret_cast<const __half*>(gptr(p.tabs[7])[e]);
    }
    const int tid = threadIdx.x, cw = tid >> 6, lane = tid & 63;
    const int g = lane >> 4, i = lane & 15, q = i & 7;
    const int ntiles = p.n >> 4;
    const int nsteps = p.ksteps;
    const int kt0 = sidx * nsteps * 4;
    const int nt = bx * 8 + cw * 2 + (i >> 3);
    const EXL3_GLOBAL uint32_t* tb = gptr(trel) + ((size_t)(kt0 + g) * ntiles + nt) * (8 * K) + K * q;
    const size_t step_stride = (size_t)4 * ntiles * (8 * K);
    const int prev_addr = ((lane & ~7) | ((lane + 7) & 7)) << 2;
    const __half2 svv = ld_h2(gptr(svh_p) + bx * 128 + 2 * lane);  // epilogue scale, requested early

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
    for (int c0 = 0; c0 < nsteps; c0 += CH) {
        // stage the chunk's A: rows x (CH * 4) slices of 16 k, permuted
        if (c0) __syncthreads();  // every wave is done with the previous chunk
        for (int u = tid; u < MT * CH * 4; u += FAT_THREADS) {
            const int row = u / (CH * 4), sl = u - row * (CH * 4);
            u32x4_t lo = {0u, 0u, 0u, 0u}, hi = {0u, 0u, 0u, 0u};
            if (row < rows && c0 * 4 + sl < nsteps * 4) {
                const EXL3_GLOBAL u32x4_t* src = reinterpret_cast<const EXL3_GLOBAL u32x4_t*>(
                    ag + (size_t)(m0 + row) * p.k + (size_t)(kt0 + c0 * 4 + sl) * 16);
                lo = src[0];
                hi = src[1];
            }
            u32x4_t* dst = reinterpret_cast<u32x4_t*>(fat_smem + (size_t)row * ROWB + sl * 32);
            dst[0] = u32x4_t{lo.x, hi.x, lo.y, hi.y};  // k pairs (0,1) (8,9) (2,3) (10,11)
            dst[1] = u32x4_t{lo.z, hi.z, lo.w, hi.w};  // k pairs (4,5) (12,13) (6,7) (14,15)
        }
        __syncthreads();

#pragma unroll
        for (int s = 0; s < CH; ++s) {
            const int step = c0 + s;
            if (step >= nsteps) break;
            const int d = step % D;
            uint32_t buf[K + 1];
#pragma unroll
            for (int j = 0; j < K; ++j) buf[1 + j] = w[d][j];
            buf[0] = (uint32_t)__builtin_amdgcn_ds_bpermute(prev_addr, (int)buf[K]);
            uint32_t frag[2][2][4];
            decode_group<K, CB, false, RAW>(buf, frag);
            if (step + D < nsteps) load_words<K>(tb + (size_t)(step + D) * step_stride, w[d]);
            const unsigned char* arow = fat_smem + (size_t)i * ROWB + (s * 4 + g) * 32;
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                if (rb * 16 >= rows) break;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const half8_t A = *reinterpret_cast<const half8_t*>(arow + (size_t)rb * 16 * ROWB + h * 16);
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
    const int c0 = bx * 128 + 2 * lane;
    if (p.gmode) {
        const float sva = __low2float(svv), svb = __high2float(svv);
        const bool clamp = p.limit > 0.0f && p.limit < __builtin_huge_valf();
        __half2 ds = __half2{};
        if (p.gmode == 2) ds = ld_h2(gptr(dsuh) + c0);
        for (int row = cw; row < rows; row += FAT_THREADS / 64) {
            float va = ct[row * 128 + 2 * lane], vb = ct[row * 128 + 2 * lane + 1];
            fwht128_pair_fast(va, vb, lane);
            va = (va * kHadNorm) * sva;
            vb = (vb * kHadNorm) * svb;
            const size_t crow = (size_t)(m0 + row);
            if (p.gmode == 1) {
                const float2 v2 = make_float2(va, vb);
                *reinterpret_cast<EXL3_GLOBAL unsigned long long*>(gptr(p.g32) + crow * p.n + c0) =
                    *reinterpret_cast<const unsigned long long*>(&v2);
            } else if (p.gmode == 2) {
                const unsigned long long gw =
                    *reinterpret_cast<const EXL3_GLOBAL unsigned long long*>(gptr(p.g32) + crow * p.n + c0);
                float ga = __uint_as_float((uint32_t)gw), gb = __uint_as_float((uint32_t)(gw >> 32));
                if (clamp) {
                    ga = fminf(ga, p.limit);
                    gb = fminf(gb, p.limit);
                    va = fminf(fmaxf(va, -p.limit), p.limit);
                    vb = fminf(fmaxf(vb, -p.limit), p.limit);
                }
                // the activation in fp16, then the down projection's input rotation of this 128-wide chunk
                const __half2 pr = __hmul2(h2_rn(silu_f(ga) * va, silu_f(gb) * vb), ds);
                float da = __low2float(pr), db = __high2float(pr);
                fwht128_pair_fast(da, db, lane);
                st_h2(gptr(p.out16) + crow * p.n + c0, h2_rn(da * kHadNorm, db * kHadNorm));
            } else {
                const int entry = gptr(p.rows_map)[crow];
                st_h2(gptr(p.out16) + (size_t)entry * p.n + c0, h2_rn(va, vb));
            }
        }
        return;
    }
    if (p.gu || p.handoff) {
        // partial-tile hand-off (gate/up mode, or plain mode with k-splits):
        // partial tile out (device-coherent stores), one counter per (column
        // block, row tile); the last of the np x S arrivals sums each row's
        // splits in split order (deterministic)
        const int np = p.gu ? 2 : 1;
        const int S = gridDim.z, proj = p.gu ? (int)(blockIdx.x & 1) : 0;
        const size_t rs = (size_t)p.M * 128;  // between splits
        float* part = p.partials + ((size_t)(bx * np + proj) * S + sidx) * rs + (size_t)m0 * 128;
        for (int idx = 2 * tid; idx < rows * 128; idx += 2 * FAT_THREADS) {
            const float2 v2 = make_float2(ct[idx], ct[idx + 1]);
            __hip_atomic_store(reinterpret_cast<unsigned long long*>(part + idx), *reinterpret_cast<const unsigned long long*>(&v2),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (p.split_out) return;  // fat_split_finish_kernel sums them
        wait_stores();
        __syncthreads();
        __shared__ int gu_last;
        int* ctr = p.counters + (size_t)bx * gridDim.y + blockIdx.y;
        if (tid == 0) {
            const int old = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            gu_last = old == np * S - 1;
        }
        __syncthreads();
        if (!gu_last) return;
        if (tid == 0) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (!p.gu) {
            const float* pv = p.partials + (size_t)bx * S * rs + (size_t)m0 * 128 + 2 * lane;
            const float sva = __low2float(svv), svb = __high2float(svv);
            if (S <= 4) {
                // the gate/up epilogue's pipelining below, one projection
                const int nchk = p.k >> 7;
                struct RowLoads1 {
                    float2 v[4];
                    float rs;
                };
                auto issue = [&](int row, RowLoads1& L) {
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        L.v[t] = t < S ? coherent_load2(pv + row * 128 + (size_t)t * rs) : make_float2(0.f, 0.f);
                    L.rs = 0.f;
                    if constexpr (RAW) {
                        const float* r = p.rowsum + (size_t)(m0 + row) * nchk;
                        for (int c = lane; c < nchk; c += 64) L.rs += gptr(r)[c];
                    }
                };
                auto consume = [&](int row, const RowLoads1& L) {
                    float va = 0.f, vb = 0.f;
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        va += L.v[t].x;
                        vb += L.v[t].y;
                    }
                    if constexpr (RAW) {
                        const float sx = kMul1Bias * wave_sum(L.rs);
                        va = va * kMul1Kinv + sx;
                        vb = vb * kMul1Kinv + sx;
                    }
                    fwht128_pair_fast(va, vb, lane);
                    st_h2(gptr(p.out16) + (size_t)(m0 + row) * p.n + c0, h2_rn((va * kHadNorm) * sva, (vb * kHadNorm) * svb));
                };
                constexpr int RS = FAT_THREADS / 64;
                RowLoads1 la, lb;
                if (cw < rows) issue(cw, la);
                for (int row = cw; row < rows; row += 2 * RS) {
                    if (row + RS < rows) issue(row + RS, lb);
                    consume(row, la);
                    if (row + RS >= rows) break;
                    if (row + 2 * RS < rows) issue(row + 2 * RS, la);
                    consume(row + RS, lb);
                }
                return;
            }
            for (int row = cw; row < rows; row += FAT_THREADS / 64) {
                const float* const src[1] = {pv + row * 128};
                float2 v2[1];
                sum_splits2<1, 4>(src, rs, S, v2);
                float va = v2[0].x, vb = v2[0].y;
                if constexpr (RAW) {
                    const float sx = kMul1Bias * fat_row_sum(p.rowsum, p.k >> 7, m0 + row, 0, p.k >> 7, lane);
                    va = va * kMul1Kinv + sx;
                    vb = vb * kMul1Kinv + sx;
                }
                fwht128_pair_fast(va, vb, lane);
                st_h2(gptr(p.out16) + (size_t)(m0 + row) * p.n + c0, h2_rn((va * kHadNorm) * sva, (vb * kHadNorm) * svb));
            }
            return;
        }
        const float* pg = p.partials + (size_t)(bx * 2) * S * rs + (size_t)m0 * 128 + 2 * lane;
        const float* pu = p.partials + (size_t)(bx * 2 + 1) * S * rs + (size_t)m0 * 128 + 2 * lane;
        const __half2 svg = ld_h2(gptr(p.svh) + c0), svu = ld_h2(gptr(p.svh2) + c0);
        // sums -> (mul1 map) -> both output rotations, svh, SwiGLU, fp16 row
        auto finish = [&](int row, float ga, float gb, float ua, float ub, float sx) {
            fat_gu_finish<RAW>(p, (size_t)(m0 + row), c0, ga, gb, ua, ub, sx, svg, svu, lane);
        };
        constexpr int RS = FAT_THREADS / 64;  // rows apart of one wave's rows
        if (S <= 4) {
            // up to 4 splits: a row's loads (both projections, every split,
            // its row sums) are requested before the wave's previous row is
            // finished, so the rows' round trips overlap (config 3 M = 16,
            // kernel alone: 26.7 -> 26.0 us).  Two named buffers keep the
            // loads in registers.
            const int nchk = p.k >> 7;
            struct RowLoads {
                float2 v[2][4];
                float rs;
            };
            auto issue = [&](int row, RowLoads& L) {
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        L.v[j][t] = t < S ? coherent_load2((j ? pu : pg) + row * 128 + (size_t)t * rs) : make_float2(0.f, 0.f);
                L.rs = 0.f;
                if constexpr (RAW) {
                    const float* r = p.rowsum + (size_t)(m0 + row) * nchk;
                    for (int c = lane; c < nchk; c += 64) L.rs += gptr(r)[c];
                }
            };
            auto consume = [&](int row, const RowLoads& L) {
                // split order, as sum_splits2
                float2 gs = make_float2(0.f, 0.f), us = make_float2(0.f, 0.f);
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    gs.x += L.v[0][t].x;
                    gs.y += L.v[0][t].y;
                    us.x += L.v[1][t].x;
                    us.y += L.v[1][t].y;
                }
                float sx = 0.f;
                if constexpr (RAW) sx = kMul1Bias * wave_sum(L.rs);
                finish(row, gs.x, gs.y, us.x, us.y, sx);
            };
            RowLoads la, lb;
            if (cw < rows) issue(cw, la);
            for (int row = cw; row < rows; row += 2 * RS) {
                if (row + RS < rows) issue(row + RS, lb);
                consume(row, la);
                if (row + RS >= rows) break;
                if (row + 2 * RS < rows) issue(row + 2 * RS, la);
                consume(row + RS, lb);
            }
            return;
        }
        for (int row = cw; row < rows; row += RS) {
            // both columns of both projections in groups of 4 splits (16
            // values and 8 addresses in flight: with 8 splits per group this
            // loop set the kernel's register budget)
            const float* const src[2] = {pg + row * 128, pu + row * 128};
            float2 gu2[2];
            sum_splits2<2, 4>(src, rs, S, gu2);
            float sx = 0.f;
            if constexpr (RAW) sx = kMul1Bias * fat_row_sum(p.rowsum, p.k >> 7, m0 + row, 0, p.k >> 7, lane);
            finish(row, gu2[0].x, gu2[0].y, gu2[1].x, gu2[1].y, sx);
        }
        return;
    }
    const float sva = __low2float(svv), svb = __high2float(svv);
    for (int row = cw; row < rows; row += FAT_THREADS / 64) {
        float va = ct[row * 128 + 2 * lane], vb = ct[row * 128 + 2 * lane + 1];
        if constexpr (RAW) {
            // this split's k range: chunks kt0 / 8 .. + nsteps / 2
            const float sx = kMul1Bias * fat_row_sum(p.rowsum, p.k >> 7, m0 + row, kt0 >> 3, nsteps >> 1, lane);
            va = va * kMul1Kinv + sx;
            vb = vb * kMul1Kinv + sx;
        }
        fwht128_pair_fast(va, vb, lane);
        va = (va * kHadNorm) * sva;
        vb = (vb * kHadNorm) * svb;
        const int src = m0 + row;
        if (p.out16) {
            st_h2(gptr(p.out16) + (size_t)src * p.n + c0, h2_rn(va, vb));
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

// Finish of the narrow kernel's split hand-off with split_out (one 16-row
// tile, up to 4 k-splits; GU: gate/up mode, else plain mode with fp16
// output): one wave per (row, column block) sums the partial rows in split
// order, from zero, as the in-kernel hand-off does, and applies the same
// epilogue, so the results are bit-identical to it.  The extra launch costs a
// kernel boundary, but every row's chain then runs at once, where the last
// arrival of a column block runs its rows on four waves behind a store /
// counter / load chain (config 3 M = 16, kernel plus finish against the
// in-kernel hand-off, graph-timed: 24.8 -> 23.4 us).
template <bool RAW, bool GU>
__global__ __launch_bounds__(256) void fat_split_finish_kernel(FatParams p, int S) {
    constexpr int NP = GU ? 2 : 1;
    const int w = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int nb = p.n >> 7;
    if (w >= nb * p.M) return;
    const int bx = w % nb, row = w / nb;
    const size_t rs = (size_t)p.M * 128;  // between splits
    const int c0 = bx * 128 + 2 * lane;
    // plain loads: the partial tiles were stored by the previous launch
    auto ld2 = [](const float* q) {
        const uint64_t u = *reinterpret_cast<const EXL3_GLOBAL uint64_t*>(gptr(q));
        return make_float2(__uint_as_float((uint32_t)u), __uint_as_float((uint32_t)(u >> 32)));
    };
    float2 v[NP][4];
#pragma unroll
    for (int j = 0; j < NP; ++j) {
        const float* pj = p.partials + (size_t)(bx * NP + j) * S * rs + (size_t)row * 128 + 2 * lane;
#pragma unroll
        for (int t = 0; t < 4; ++t) v[j][t] = t < S ? ld2(pj + (size_t)t * rs) : make_float2(0.f, 0.f);
    }
    const __half2 sv0 = ld_h2(gptr(p.svh) + c0);
    const __half2 sv1 = GU ? ld_h2(gptr(p.svh2) + c0) : sv0;
    float rsum = 0.f;
    if constexpr (RAW) {
        const int nchk = p.k >> 7;
        const float* r = p.rowsum + (size_t)row * nchk;
        for (int c = lane; c < nchk; c += 64) rsum += gptr(r)[c];
    }
    float2 sm[NP];
#pragma unroll
    for (int j = 0; j < NP; ++j) {
        sm[j] = make_float2(0.f, 0.f);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            sm[j].x += v[j][t].x;
            sm[j].y += v[j][t].y;
        }
    }
    float sx = 0.f;
    if constexpr (RAW) sx = kMul1Bias * wave_sum(rsum);
    if constexpr (GU) {
        fat_gu_finish<RAW>(p, (size_t)row, c0, sm[0].x, sm[0].y, sm[NP - 1].x, sm[NP - 1].y, sx, sv0, sv1, lane);
    } else {
        float va = sm[0].x, vb = sm[0].y;
        if constexpr (RAW) {
            va = va * kMul1Kinv + sx;
            vb = vb * kMul1Kinv + sx;
        }
        fwht128_pair_fast(va, vb, lane);
        st_h2(gptr(p.out16) + (size_t)row * p.n + c0,
              h2_rn((va * kHadNorm) * __low2float(sv0), (vb * kHadNorm) * __high2float(sv0)));
    }
}

// ------------------------------------------------------------ wide tiles
//
// MFMA-bound shapes (many rows).  A workgroup of 8 waves owns 256 rows x 256
// columns: wave (rh, cq) computes rows 128rh .. +128 x columns 64cq .. +64
// (row blocks x two 32-column decode groups per lane).  The two waves of a
// column quarter share its decode: wave rh decodes group G = rh of the next
// step and posts the MFMA B fragments in LDS; both read both groups back.  So
// each decoded weight feeds 256 rows at half a 64-column decode per wave, and
// each staged A fragment feeds four MFMAs.  Two waves per SIMD, 128
// accumulators each.  (On gfx950 VALU and MFMA work barely overlap: the
// decode's VALU time adds to the MFMA time, so it is cut per MAC.)
//
// A is staged one step (64 k) at a time into two LDS buffers: each thread
// loads four 16-byte chunks of the next step into registers after its decode
// and writes them after its MFMAs, in natural k order with the 16-byte chunk
// index XOR-swizzled by row (chunk ^ (row & 7) ^ ((row >> 3) & 1)), which
// keeps the fragment reads conflict-free for 8- and 16-lane LDS phases.
// (Direct global->LDS loads measured slower, and the compiler's vmcnt
// tracking does not see them, forcing full waits.)  Natural k order works
// because each lane decodes all 16 k values of its two columns: fragment word
// j of run h' is tile rows (8h' + 2j, 8h' + 2j + 1).  B fragments sit
// chunk-major ([quarter][group][chunk][lane] x 16 bytes), so their 16-byte
// writes and reads are conflict-free too.
//
// Step s: request the A chunks of step s+1; phase A: the row-half-0 waves
// run the step's 64 MFMAs on the current buffers while the row-half-1 waves
// decode their group of step s+1 into the other B buffer and request the
// weights of step s+2; phase B: the same with the roles swapped; then the A
// chunks are written.  Two barriers per step, which wait for the LDS traffic
// only.
constexpr int FB_ROWS = 256;
constexpr int FB_COLS = 256;
constexpr int FB_THREADS = 512;                 // 8 waves: 2 row halves x 4 column quarters
constexpr int FB_A_BYTES = FB_ROWS * 128;       // one staged step: 256 rows x 64 k fp16
constexpr int FB_B_BYTES = 4 * 2 * 4 * 64 * 16;  // one step's B fragments: [quarter][group][chunk][lane]
constexpr int FB_PASS_ROWS = 64;                // epilogue rows per LDS pass (32 of each half)
constexpr int FB_CTS = FB_COLS + 4;             // epilogue row stride (floats)
constexpr int FAT_MT_WIDE = 0;                  // plan value (rows per tile) selecting fat_big_kernel
constexpr int FB_TAIL_FLOATS = FB_ROWS * FB_COLS;  // one tile's fp32 accumulators (tail split)

constexpr size_t fat_big_smem_bytes() {
    constexpr size_t stage = 2 * (size_t)FB_A_BYTES + 2 * (size_t)FB_B_BYTES;
    constexpr size_t tile = (size_t)FB_PASS_ROWS * FB_CTS * sizeof(float);
    return stage > tile ? stage : tile;
}

// fp16 pair of tile rows (4H + kofs(2P), +1) of column q + 8C (round to
// nearest; RAW: the mul1 raw entries of mul1_raw_pair).
template <int K, int CB, int H, int C, int P, bool RAW = false>
__device__ __forceinline__ uint32_t nat_pair(const uint32_t* buf, const uint32_t* mid) {
    constexpr int e0 = 2 * P, e1 = 2 * P + 1;
    constexpr int u0 = 16 * H + (e0 & 3) + 8 * (e0 >> 2) + 4 * C;
    constexpr int u1 = 16 * H + (e1 & 3) + 8 * (e1 >> 2) + 4 * C;
    if constexpr (RAW) {
        static_assert(CB == 2, "raw entries: mul1");
        return mul1_raw_pair(window_mid<K, u0>(buf, mid), window_mid<K, u1>(buf, mid));
    } else {
        return decode2_rn<CB>(window_mid<K, u0>(buf, mid), window_mid<K, u1>(buf, mid));
    }
}

// f[h'][j] = tile rows (8h' + 2j, +1) of column q + 8C: run H = j >> 1, pair P = h' + 2 (j & 1).
template <int K, int CB, int C, bool RAW>
__device__ __forceinline__ void nat_column(const uint32_t* buf, const uint32_t* mid, uint32_t (&f)[2][4]) {
    f[0][0] = nat_pair<K, CB, 0, C, 0, RAW>(buf, mid);
    f[0][1] = nat_pair<K, CB, 0, C, 2, RAW>(buf, mid);
    f[0][2] = nat_pair<K, CB, 1, C, 0, RAW>(buf, mid);
    f[0][3] = nat_pair<K, CB, 1, C, 2, RAW>(buf, mid);
    f[1][0] = nat_pair<K, CB, 0, C, 1, RAW>(buf, mid);
    f[1][1] = nat_pair<K, CB, 0, C, 3, RAW>(buf, mid);
    f[1][2] = nat_pair<K, CB, 1, C, 1, RAW>(buf, mid);
    f[1][3] = nat_pair<K, CB, 1, C, 3, RAW>(buf, mid);
}

// Decode one 32-value group (words w[0..K-1], previous word from lane q - 1).
template <int K, int CB, bool RAW = false>
__device__ __forceinline__ void nat_group(const uint32_t (&w)[K], int prev_addr, uint32_t (&f)[2][2][4]) {
    uint32_t buf[K + 1], mid[K];
#pragma unroll
    for (int j = 0; j < K; ++j) buf[1 + j] = w[j];
    buf[0] = (uint32_t)__builtin_amdgcn_ds_bpermute(prev_addr, (int)buf[K]);
#pragma unroll
    for (int j = 0; j < K; ++j) mid[j] = __builtin_amdgcn_alignbit(buf[j], buf[j + 1], 16);
    nat_column<K, CB, 0, RAW>(buf, mid, f[0]);
    nat_column<K, CB, 1, RAW>(buf, mid, f[1]);
}

// mul1 raw entries in the x16 layout (a tile row on 8 lanes, 16 columns
// each): kMul1Bias * S, S the sum of the row's x over chunks [c0, c0 + nc)
// of rowsum (lane j of the 8 adds chunks j, j + 8, .., then the 8 partials
// meet by DPP), and the correction v = v * kMul1Kinv + that term.
__device__ __forceinline__ float raw_row_bias(const FatParams& p, int row, int c0, int nc, int lane) {
    const float* r = p.rowsum + (size_t)row * (p.k >> 7) + c0;
    float t = 0.f;
    for (int c = lane & 7; c < nc; c += 8) t += gptr(r)[c];
    t += lane_xor<1>(t);
    t += lane_xor<2>(t);
    t += lane_xor<4>(t);
    return kMul1Bias * t;
}
__device__ __forceinline__ void raw_fix16(float (&v)[16], float sx) {
#pragma unroll
    for (int e = 0; e < 16; ++e) v[e] = v[e] * kMul1Kinv + sx;
}

// GU = true: gate/up mode.  Workgroup bx then covers column block bx of both
// projections: its left 128 columns (column quarters 0, 1) decode the gate
// trellis, its right 128 (quarters 2, 3) the up trellis, so the epilogue
// holds the gate and up values of the same columns and applies the SwiGLU
// in registers.  The reference's fused path concatenates the two packs per
// call and combines them with separate torch kernels
// (src/sglang_exl3/exl3.py:1184-1206).
// RAW (mul1, p.rowsum set): B holds the raw entries (mul1_raw_pair) and the
// epilogue applies kMul1Kinv * acc + kMul1Bias * (the row's x sum over the
// k range) before the output rotation, two VALU per pair of states fewer in
// the decode (config 3 M = 2048, whole-tile harness: 497.6 -> 483.2 us).
template <int K, int CB, bool GU, bool RAW = false>
__global__ __launch_bounds__(FB_THREADS, 2) void fat_big_kernel(FatParams p) {
    constexpr int RB = FB_ROWS / 2 / 16;  // row blocks per wave
    static_assert(FB_A_BYTES == 4 * 16 * FB_THREADS, "four 16-byte A chunks per thread and step");
    extern __shared__ __align__(16) unsigned char fat_smem[];
    unsigned char* const bsm = fat_smem + 2 * FB_A_BYTES;

    // tile of this workgroup (and, tail split, which k-half of it: -1 whole)
    int bx = blockIdx.x, by = blockIdx.y, half = -1, slot = 0;
    if (p.tail_tiles > 0) {
        int lin = blockIdx.x;
        if (lin >= p.tail_first) {
            slot = (lin - p.tail_first) >> 1;
            half = (lin - p.tail_first) & 1;
            lin = p.tail_first + slot;
        }
        // wave-uniform: kept in scalar registers
        by = __builtin_amdgcn_readfirstlane(lin / p.tiles_x);
        bx = __builtin_amdgcn_readfirstlane(lin - by * p.tiles_x);
        half = __builtin_amdgcn_readfirstlane(half);
        slot = __builtin_amdgcn_readfirstlane(slot);
    }
    const int sidx = blockIdx.z;
    const int m0 = by * FB_ROWS;
    const int rows = min(FB_ROWS, p.M - m0);
    const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
    const int rh = wv >> 2, cq = wv & 3;
    const int g = lane >> 4, i = lane & 15, q = i & 7;
    const int ntiles = p.n >> 4;
    const int nsteps = half >= 0 ? p.ksteps / 2 : p.ksteps;  // even
    const int kt0 = sidx * p.ksteps * 4 + (half > 0 ? nsteps * 4 : 0);
    // this wave decodes group rh of quarter cq: column tiles 4cq + 2rh + (i >> 3)
    // (gate/up mode: quarters 0, 1 of the gate block bx, 2, 3 of the up block bx)
    const int nt = GU ? bx * 8 + (cq & 1) * 4 + rh * 2 + (i >> 3) : bx * (FB_COLS / 16) + cq * 4 + rh * 2 + (i >> 3);
    const uint32_t* trel = (GU && cq >= 2) ? p.trellis2 : p.trellis;
    const EXL3_GLOBAL uint32_t* tb = gptr(trel) + ((size_t)(kt0 + g) * ntiles + nt) * (8 * K) + K * q;
    const size_t step_stride = (size_t)4 * ntiles * (8 * K);
    const int prev_addr = ((lane & ~7) | ((lane + 7) & 7)) << 2;

    // A staging: thread t moves chunks u = t + 512j (j < 4): tile row u >> 3,
    // physical chunk u & 7, which holds logical chunk (u & 7) ^ (row & 7) ^
    // ((row >> 3) & 1).  Rows past M repeat the last row (never stored).
    const EXL3_GLOBAL char* abase =
        reinterpret_cast<const EXL3_GLOBAL char*>(gptr(p.a)) + ((size_t)m0 * p.k + (size_t)kt0 * 16) * 2;
    uint32_t aoff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int u = tid + FB_THREADS * j;
        const int row = min(u >> 3, rows - 1);
        const int c = (u & 7) ^ ((u >> 3) & 7) ^ ((u >> 6) & 1);
        aoff[j] = (uint32_t)row * (uint32_t)p.k * 2u + 16u * (uint32_t)c;
    }
    u32x4_t areg[4];
    auto load_a = [&](int step) {
        const EXL3_GLOBAL char* src = abase + (size_t)step * 128;
#pragma unroll
        for (int j = 0; j < 4; ++j) areg[j] = *reinterpret_cast<const EXL3_GLOBAL u32x4_t*>(src + aoff[j]);
    };
    auto write_a = [&](int bufi) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            *reinterpret_cast<u32x4_t*>(fat_smem + (size_t)bufi * FB_A_BYTES + (size_t)(tid + FB_THREADS * j) * 16) =
                areg[j];
    };
    // A fragment reads: row 128rh + 16rb + i, logical chunk 2g + h'
    uint32_t rd_off[2];
#pragma unroll
    for (int h = 0; h < 2; ++h)
        rd_off[h] = (uint32_t)(rh * 128 + i) * 128u + 16u * (uint32_t)((2 * g + h) ^ (i & 7) ^ (i >> 3));
    // B fragments: chunk (c, h') of group G of this quarter
    auto b_off = [&](int G, int c, int h) { return (uint32_t)(((cq * 2 + G) * 4 + c * 2 + h) * 1024 + lane * 16); };

    float4_t acc[RB][2][2];  // [row block][group][column half]
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int G = 0; G < 2; ++G)
#pragma unroll
            for (int c = 0; c < 2; ++c) acc[rb][G][c] = float4_t{0.f, 0.f, 0.f, 0.f};

    uint32_t w[K];  // this wave's words of the next step to decode
    auto load_step = [&](int step) { load_words<K>(tb + (size_t)step * step_stride, w); };
    auto decode_post = [&](int bufi) {
        uint32_t fr[2][2][4];  // [column half][h'][j]
        nat_group<K, CB, RAW>(w, prev_addr, fr);
        unsigned char* bb = bsm + (size_t)bufi * FB_B_BYTES;
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                *reinterpret_cast<u32x4_t*>(bb + b_off(rh, c, h)) = u32x4_t{fr[c][h][0], fr[c][h][1], fr[c][h][2], fr[c][h][3]};
    };

    load_step(0);
    load_a(0);
    write_a(0);
    __syncthreads();
    decode_post(0);
    load_step(nsteps > 1 ? 1 : 0);
    __syncthreads();

    // buffers SL = s & 1 hold step s; requests past the last step are clamped
    // to it (no branch inside the unrolled body; the extra decode is unused)
    auto mfma_phase = [&](auto slot_c) {
        constexpr int SL = decltype(slot_c)::value;
        const unsigned char* ab = fat_smem + (size_t)SL * FB_A_BYTES;
        const unsigned char* bb = bsm + (size_t)SL * FB_B_BYTES;
        half8_t B[2][2][2];  // [group][column half][h']
#pragma unroll
        for (int G = 0; G < 2; ++G)
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int h = 0; h < 2; ++h) B[G][c][h] = *reinterpret_cast<const half8_t*>(bb + b_off(G, c, h));
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const half8_t A = *reinterpret_cast<const half8_t*>(ab + rd_off[h] + rb * 2048);
#pragma unroll
                for (int G = 0; G < 2; ++G)
#pragma unroll
                    for (int c = 0; c < 2; ++c)
                        acc[rb][G][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B[G][c][h], acc[rb][G][c], 0, 0, 0);
            }
        }
    };
    // Ping-pong: each step has two phases, one barrier after each.  In phase A
    // the row-half-0 waves run the step's MFMAs while the row-half-1 waves
    // decode their group of step s+1; in phase B the roles swap.  The two
    // waves of a SIMD (the same column quarter) are then never in the same
    // role, so one's decode and the other's MFMAs share the SIMD instead of
    // both waves decoding, then both multiplying (config 3 M=2048, graph-timed
    // on one box: 547 -> 528 us).  A chunks of step s+1 are requested at the
    // start of step s and written after phase B; the B buffer a phase writes
    // was last read in the step before (both phases).  Decode and MFMA code
    // are kept apart (sched_barrier): mixing them raises register pressure
    // past the 256 of two waves per SIMD.
    auto run_mfma = [&](auto slot_c) {
        if constexpr (EXL3_FAT_SETPRIO) __builtin_amdgcn_s_setprio(1);
        mfma_phase(slot_c);
        if constexpr (EXL3_FAT_SETPRIO) __builtin_amdgcn_s_setprio(0);
    };
    auto step_body = [&](int s, auto slot_c) {
        constexpr int SL = decltype(slot_c)::value;
        const int n1 = s + 1 < nsteps ? s + 1 : s;
        const int n2 = s + 2 < nsteps ? s + 2 : n1;
        load_a(n1);
        if (rh == 0) {  // phase A
            run_mfma(slot_c);
        } else {
            decode_post(SL ^ 1);
            load_step(n2);
        }
        __builtin_amdgcn_sched_barrier(0);
        // A barrier on the LDS traffic only (__syncthreads would also wait for
        // the weight request, which the next decode waits for by itself).
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        if (rh != 0) {  // phase B
            run_mfma(slot_c);
        } else {
            decode_post(SL ^ 1);
            load_step(n2);
        }
        __builtin_amdgcn_sched_barrier(0);
        write_a(SL ^ 1);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
    };
    for (int s = 0; s < nsteps; s += 2) {
        step_body(s, std::integral_constant<int, 0>{});
        step_body(s + 1, std::integral_constant<int, 1>{});
    }
    __syncthreads();  // everything landed before the epilogue reuses the LDS

    if (half >= 0) {
        // tail split: the first half to get here hands its accumulators to
        // the second (one device-coherent store and load per value; fp32
        // addition is commutative, so the sum does not depend on which half
        // came first)
        __shared__ int tail_old;
        if (tid == 0) tail_old = __hip_atomic_fetch_add(p.tail_sync + slot, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        // pair j of thread t at [j][t]: each store covers 512 consecutive bytes
        unsigned long long* part = reinterpret_cast<unsigned long long*>(p.tail_part + (size_t)slot * FB_TAIL_FLOATS) + tid;
        int* flag = p.tail_sync + p.tail_tiles + slot;
        if (tail_old == 0) {
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int G = 0; G < 2; ++G)
#pragma unroll
                    for (int c = 0; c < 2; ++c)
#pragma unroll
                        for (int h = 0; h < 2; ++h) {
                            const int j = ((rb * 2 + G) * 2 + c) * 2 + h;
                            const float2 v = make_float2(acc[rb][G][c][2 * h], acc[rb][G][c][2 * h + 1]);
                            __hip_atomic_store(part + (size_t)j * FB_THREADS, *reinterpret_cast<const unsigned long long*>(&v),
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        }
            wait_stores();
            __syncthreads();
            if (tid == 0) __hip_atomic_store(flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
        if (tid == 0) {
            // bounded (p.max_polls polls of ~0.2 us each) so that every wave
            // exits even if the first half never stored; a wait that gives
            // up is reported in the workspace status word
            bool got = false;
            for (int it = 0; it < p.max_polls; ++it) {
                if (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
                    got = true;
                    break;
                }
                __builtin_amdgcn_s_sleep(8);
            }
            if (!got) report_wait_expired(p.status, EXL3_WAIT_FAT_TAIL);
            __hip_atomic_store(p.tail_sync + slot, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(flag, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        // the first half's sums are added as the epilogue moves the
        // accumulators to LDS (adding them into the accumulators here would
        // keep a second copy of all 128 live)
    }
    const unsigned long long* tail_other =
        half >= 0 ? reinterpret_cast<const unsigned long long*>(p.tail_part + (size_t)slot * FB_TAIL_FLOATS) + tid
                  : nullptr;

    // epilogue: 4 passes through LDS, pass p holding tile rows 32p .. +32 of
    // each half (LDS row rh*32 + local); the output FWHT, norm and svh per
    // (row, 128-block).  Accumulator (rb, G, c, r) is tile row
    // 128rh + 16rb + 4g + r, column 64cq + 32G + 16(i >> 3) + (i & 7) + 8c.
    float* ct = reinterpret_cast<float*>(fat_smem);
#pragma unroll
    for (int pass = 0; pass < RB / 2; ++pass) {
        if (pass * 32 >= rows) break;
        if (pass) __syncthreads();
#pragma unroll
        for (int rr = 0; rr < 2; ++rr)
#pragma unroll
            for (int G = 0; G < 2; ++G)
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    float o[4] = {0.f, 0.f, 0.f, 0.f};
                    if (tail_other) {
                        const int j = (((pass * 2 + rr) * 2 + G) * 2 + c) * 2;
                        const unsigned long long u0 = __hip_atomic_load(tail_other + (size_t)j * FB_THREADS,
                                                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        const unsigned long long u1 = __hip_atomic_load(tail_other + (size_t)(j + 1) * FB_THREADS,
                                                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        o[0] = __uint_as_float((uint32_t)u0);
                        o[1] = __uint_as_float((uint32_t)(u0 >> 32));
                        o[2] = __uint_as_float((uint32_t)u1);
                        o[3] = __uint_as_float((uint32_t)(u1 >> 32));
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int row = rh * 32 + rr * 16 + 4 * g + r;
                        const int col = cq * 64 + G * 32 + (i >> 3) * 16 + (i & 7) + 8 * c;
                        ct[row * FB_CTS + col] = acc[pass * 2 + rr][G][c][r] + o[r];
                    }
                }
        __syncthreads();
        if constexpr (GU) {
            // 8 rows per wave, gate and up of one 128-column block: lane l
            // holds 16 consecutive columns (16 (l & 7) ..) of each, LDS row
            // 8 wv + (l >> 3); output FWHT, norm and svh of both, then SwiGLU
            static_assert(FB_PASS_ROWS / 8 == FB_THREADS / 64, "one row group per wave");
            const int ctr = wv * 8 + (lane >> 3);
            const int trow = (ctr >> 5) * 128 + pass * 32 + (ctr & 31);
            const int col = (lane & 7) * 16;
            float gv[16], uv[16];
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const float4 a = *reinterpret_cast<const float4*>(ct + ctr * FB_CTS + col + 4 * q4);
                const float4 b = *reinterpret_cast<const float4*>(ct + ctr * FB_CTS + 128 + col + 4 * q4);
                gv[4 * q4] = a.x; gv[4 * q4 + 1] = a.y; gv[4 * q4 + 2] = a.z; gv[4 * q4 + 3] = a.w;
                uv[4 * q4] = b.x; uv[4 * q4 + 1] = b.y; uv[4 * q4 + 2] = b.z; uv[4 * q4 + 3] = b.w;
            }
            if constexpr (RAW) {
                const float sx = raw_row_bias(p, m0 + (trow < rows ? trow : rows - 1), sidx * (p.ksteps >> 1),
                                              p.ksteps >> 1, lane);
                raw_fix16(gv, sx);
                raw_fix16(uv, sx);
            }
            fwht128_x16(gv, lane);
            fwht128_x16(uv, lane);
            const float hn = fwht_x16_norm(lane);
            const int c0 = bx * 128 + col;
            const EXL3_GLOBAL uint32_t* sgp = reinterpret_cast<const EXL3_GLOBAL uint32_t*>(gptr(p.svh) + c0);
            const EXL3_GLOBAL uint32_t* sup = reinterpret_cast<const EXL3_GLOBAL uint32_t*>(gptr(p.svh2) + c0);
#pragma unroll
            for (int e2 = 0; e2 < 8; ++e2) {
                const uint32_t sgw = sgp[e2], suw = sup[e2];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int e = 2 * e2 + h;
                    gv[e] = (gv[e] * hn) * __half2float(__ushort_as_half((unsigned short)(sgw >> (16 * h))));
                    uv[e] = (uv[e] * hn) * __half2float(__ushort_as_half((unsigned short)(suw >> (16 * h))));
                }
            }
            // one uniform branch around all 32 values: a per-value test is
            // turned into selects that cost 80 VALU per pass without a clamp
            if (p.limit > 0.0f && p.limit < __builtin_huge_valf()) {
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    gv[e] = fminf(gv[e], p.limit);
                    uv[e] = fminf(fmaxf(uv[e], -p.limit), p.limit);
                }
            }
            uint32_t ow[8];
#pragma unroll
            for (int e2 = 0; e2 < 8; ++e2) {
                const __half2 o = h2_rn(silu_f(gv[2 * e2]) * uv[2 * e2], silu_f(gv[2 * e2 + 1]) * uv[2 * e2 + 1]);
                ow[e2] = *reinterpret_cast<const uint32_t*>(&o);
            }
            if (trow < rows) {
                EXL3_GLOBAL uint32_t* o = reinterpret_cast<EXL3_GLOBAL uint32_t*>(gptr(p.out16) + (size_t)(m0 + trow) * p.n + c0);
#pragma unroll
                for (int e2 = 0; e2 < 8; ++e2) o[e2] = ow[e2];
            }
            continue;
        }
        // 8 rows x one 128-block per wave at a time: lane l holds 16 consecutive
        // columns (16 (l & 7) ..) of LDS row 8 rg + (l >> 3)
#pragma unroll
        for (int gi = wv; gi < FB_PASS_ROWS / 8 * (FB_COLS / 128); gi += FB_THREADS / 64) {
            const int b = gi & 1, rg = gi >> 1;
            const int ctr = rg * 8 + (lane >> 3);
            const int trow = (ctr >> 5) * 128 + pass * 32 + (ctr & 31);
            const int col = b * 128 + (lane & 7) * 16;
            float v[16];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 t = *reinterpret_cast<const float4*>(ct + ctr * FB_CTS + col + 4 * q);
                v[4 * q] = t.x;
                v[4 * q + 1] = t.y;
                v[4 * q + 2] = t.z;
                v[4 * q + 3] = t.w;
            }
            if constexpr (RAW)
                raw_fix16(v, raw_row_bias(p, m0 + (trow < rows ? trow : rows - 1), sidx * (p.ksteps >> 1),
                                          p.ksteps >> 1, lane));
            fwht128_x16(v, lane);
            const float hn = fwht_x16_norm(lane);
            const int c0 = bx * FB_COLS + col;
            // svh and the outputs are only 4- (8-) byte aligned by contract
            const EXL3_GLOBAL uint32_t* svp = reinterpret_cast<const EXL3_GLOBAL uint32_t*>(gptr(p.svh) + c0);
            uint32_t sw[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) sw[e] = svp[e];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const __half sv = __ushort_as_half((unsigned short)(sw[e >> 1] >> (16 * (e & 1))));
                v[e] = (v[e] * hn) * __half2float(sv);
            }
            if (p.accumulate) {
                // atomics want a wave's lanes on consecutive columns: the
                // transformed rows go back to LDS (this wave's own rows) and
                // leave as (row, 2 columns per lane) pairs
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    *reinterpret_cast<float4*>(ct + ctr * FB_CTS + col + 4 * q) =
                        make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
#pragma unroll
                for (int r8 = 0; r8 < 8; ++r8) {
                    const int cr = rg * 8 + r8;
                    const int tr = (cr >> 5) * 128 + pass * 32 + (cr & 31);
                    if (tr >= rows) continue;
                    const float2 pv = *reinterpret_cast<const float2*>(ct + cr * FB_CTS + b * 128 + 2 * lane);
                    const int src = m0 + tr;
                    size_t dst = (size_t)src;
                    if (p.token_idx) dst = (size_t)gptr(p.token_idx)[src];
                    float rw = 1.f;
                    if (p.route_w)
                        rw = __half2float(__ushort_as_half(gptr(reinterpret_cast<const uint16_t*>(p.route_w))[src]));
                    float* o = p.out32 + dst * p.n + bx * FB_COLS + b * 128 + 2 * lane;
                    atomicAdd(o, pv.x * rw);
                    atomicAdd(o + 1, pv.y * rw);
                }
                continue;
            }
            if (trow >= rows) continue;
            const int src = m0 + trow;
            if (p.out16) {
                __half* o = p.out16 + (size_t)src * p.n + c0;
#pragma unroll
                for (int e = 0; e < 8; ++e) st_h2(gptr(o) + 2 * e, h2_rn(v[2 * e], v[2 * e + 1]));
                continue;
            }
            float* o = p.out32 + (size_t)src * p.n + c0;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float2 v2 = make_float2(v[2 * e], v[2 * e + 1]);
                reinterpret_cast<EXL3_GLOBAL unsigned long long*>(gptr(o))[e] =
                    *reinterpret_cast<const unsigned long long*>(&v2);
            }
        }
    }
}

template <int K>
int fat_launch_k(int cb, int mt, const FatParams& p, int splits, hipStream_t st) {
    if (mt == FAT_MT_WIDE) {
        dim3 grid(p.gu ? p.n / 128 : p.n / FB_COLS, (p.M + FB_ROWS - 1) / FB_ROWS, splits);
        if (p.tail_tiles > 0) grid = dim3(p.tail_first + 2 * p.tail_tiles, 1, 1);
        const size_t smem = fat_big_smem_bytes();
#define EXL3_FATB(CBV, GUV, RAWV)                                                                      \
    if (cb == CBV && (p.gu != 0) == GUV && (p.rowsum != nullptr) == RAWV) {                            \
        const void* fn = reinterpret_cast<const void*>(&fat_big_kernel<K, CBV, GUV, RAWV>);            \
        const int lrc = allow_dynamic_lds(fn, smem, "exl3 fat gemm (wide tiles)");                     \
        if (lrc) return lrc;                                                                           \
        fat_big_kernel<K, CBV, GUV, RAWV><<<grid, FB_THREADS, smem, st>>>(p);                          \
        return launch_status("exl3 fat gemm launch");                                                  \
    }
        EXL3_FATB(0, false, false) EXL3_FATB(1, false, false) EXL3_FATB(2, false, false)
        EXL3_FATB(0, true, false) EXL3_FATB(1, true, false) EXL3_FATB(2, true, false)
        EXL3_FATB(2, true, true)
#undef EXL3_FATB
    }
    dim3 grid((p.gu ? 2 : 1) * (p.n / 128), (p.M + mt - 1) / mt, splits);
    const size_t smem = fat_smem_bytes(mt);
#define EXL3_FAT_R(CBV, MTV, RAWV)                                                                     \
    if (cb == CBV && mt == MTV && (p.rowsum != nullptr) == RAWV) {                                     \
        const void* fn = reinterpret_cast<const void*>(&fat_gemm_kernel<K, CBV, MTV, RAWV>);           \
        const int lrc = allow_dynamic_lds(fn, smem, "exl3 fat gemm");                                  \
        if (lrc) return lrc;                                                                           \
        fat_gemm_kernel<K, CBV, MTV, RAWV><<<grid, FAT_THREADS, smem, st>>>(p);                        \
        return launch_status("exl3 fat gemm launch");                                                  \
    }
#define EXL3_FAT(CBV, MTV) EXL3_FAT_R(CBV, MTV, false)
#define EXL3_FAT_CB(CBV) EXL3_FAT(CBV, 16) EXL3_FAT(CBV, 64) EXL3_FAT(CBV, 128)
    EXL3_FAT_CB(0) EXL3_FAT_CB(1) EXL3_FAT_CB(2)
    // mul1 raw entries: 16-row tiles, plain and gate/up modes
    if (!p.gmode) { EXL3_FAT_R(2, 16, true) }
#undef EXL3_FAT_CB
#undef EXL3_FAT
#undef EXL3_FAT_R
    set_error("exl3 fat gemm: no kernel for codebook %d tile rows %d", cb, mt);
    return EXL3_ERR_UNSUPPORTED;
}

// One instantiation unit per K (exl3_fat_inst.hip built with -DEXL3_K=K).
int fat_launch(int K, int cb, int mt, const FatParams& p, int splits, hipStream_t st);

}  // namespace exl3
