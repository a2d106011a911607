// Small-m EXL3 GEMV / skinny GEMM kernel for gfx950 (one launch per call).
//
//   y = svh (.) H( x' . T ) / sqrt(128),   x' = fp16( H( fp16(x (.) suh) ) / sqrt(128) )
//
// Reference semantics: csrc/quant/exl3_gemv_kernel.cuh:138-402 (input
// rotation, decode + product, k-split reduce, output rotation).
//
// Layout of the work:
//   grid = (n/128 column blocks, S k-splits, E experts); a workgroup has
//   4*KW waves: wave w owns output columns [32(w%4), +32) of the block and the
//   (w/4)-th of KW consecutive k ranges of the split.  Per step a wave covers
//   4 k-slices x 2 column tiles: lane L = 16g + i decodes group q = i%8 of
//   tile (kt + g, nt0 + i/8) -> 32 "pair-form" words (two fp16 numbers each,
//   see exl3_decode.h) = 8 MFMA B fragments (2 columns x 4 quarters of k).
//   The activation x' is staged in LDS in the matching A-fragment order with
//   every value duplicated into both halves of a word, so each
//   v_mfma_f32_16x16x32_f16 adds x'*(lo + hi) exactly in fp32.
//   Activation loads are issued before the weight loads, and all weight loads
//   of a wave are in flight while the input rotation runs.
//   k ranges of the KW waves are summed through LDS; k-split partial sums go
//   to the workspace through device-coherent stores; the last workgroup of a
//   column block (atomic counter, self-resetting) sums them in split order
//   (deterministic), applies the output FWHT and svh, and stores fp16.
#pragma once

#include "exl3_common.h"
#include "exl3_decode.h"

namespace exl3 {

constexpr int GV_MAX_THREADS = 512;  // 4 column waves x up to 2 k waves
constexpr int GV_PRE = 8;            // rotation blocks per wave whose activations are preloaded

struct GemvParams {
    const __half* x;
    long long x_stride_e;  // elements between consecutive experts' x (0 = shared x)
    const uint32_t* trellis;
    const __half* suh;
    const __half* svh;
    const int64_t* t_tab;  // batched form: per-expert pointer tables + ids
    const int64_t* su_tab;
    const int64_t* sv_tab;
    const int32_t* ids;
    __half* y;
    long long y_stride_e;
    float* partials;  // [E][n/128][S][m][128]
    int* counters;    // [E][n/128]
    int m, k, n;
    int nsteps;  // steps (4 k-slices each) per wave
    int kw;      // waves along k inside a workgroup (1 or 2)
    int splits;  // S: workgroups along k
    // Gate/up mode (two "experts" on grid.z: 0 = gate with trellis/suh/svh,
    // 1 = up with trellis2/suh2/svh2): the 2 S workgroups of a column block
    // share one counter, and the last of them writes
    // y[row][col] = fp16( silu(min(g, limit)) * clamp(u, -limit, limit) ).
    int gu;
    const uint32_t* trellis2;
    const __half* suh2;
    const __half* svh2;
    float limit;
    // x holds the rows already rotated (x (.) suh, FWHT, / sqrt(128), fp16;
    // rotate_rows_kernel): the workgroups stage them as they are
    int x_rot;
    // k-split hand-off in one round trip (fx != 0, gemv_kernel<.., FX = true>,
    // one matrix): every split rotates and scales its own partial rows and
    // adds them into the 64-bit fixed-point accumulators acc[m][n] (zero
    // between calls; the format of the balanced kernel), and the add that
    // completes an element's `splits` contributions writes its fp16 value
    // and clears the accumulator (the output rotation is linear).
    int fx;
    unsigned long long* acc;
};

// Steps of weight words a wave keeps in flight.  Measured on MI355X (config 2,
// m=1): depth 2 is as fast as 4, 6 or 8 at every launch shape and the fastest
// at the planner's shape; the fewer registers keep occupancy up.
template <int K>
__host__ __device__ constexpr int gv_depth() {
    return 2;
}

// fp16 pair from global memory (loaded as a 32-bit word).
__device__ __forceinline__ __half2 ld_h2(const EXL3_GLOBAL __half* p) {
    const uint32_t u = *reinterpret_cast<const EXL3_GLOBAL uint32_t*>(p);
    return *reinterpret_cast<const __half2*>(&u);
}
__device__ __forceinline__ void st_h2(EXL3_GLOBAL __half* p, __half2 v) {
    *reinterpret_cast<EXL3_GLOBAL uint32_t*>(p) = *reinterpret_cast<const uint32_t*>(&v);
}

// Device-coherent (sc1) store/load: visible to every workgroup of the device
// without an L2 write-back / invalidate.
__device__ __forceinline__ void coherent_store(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float coherent_load(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Two adjacent floats through one device-coherent 8-byte load.
__device__ __forceinline__ float2 coherent_load2(const float* p) {
    const unsigned long long u = __hip_atomic_load(reinterpret_cast<unsigned long long*>(const_cast<float*>(p)),
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return make_float2(__uint_as_float((uint32_t)u), __uint_as_float((uint32_t)(u >> 32)));
}

// A bounded wait gave up: OR `bit` (EXL3_WAIT_*) into the workspace status
// word, where exl3_workspace_status finds it.
__device__ __forceinline__ void report_wait_expired(int* status, int bit) {
    __hip_atomic_fetch_or(status, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

constexpr int GV_MAX_SPLITS = 16;  // k-splits a reduction reads in one round trip

// sum_{s < S} p[s * stride] in split order.  The S device-coherent loads are
// all issued before the first add, so the reduction costs one memory round
// trip instead of S (S <= GV_MAX_SPLITS; larger S continues in groups).
__device__ __forceinline__ float sum_splits(const float* p, size_t stride, int S) {
    float sum = 0.f;
    for (int s0 = 0; s0 < S; s0 += GV_MAX_SPLITS) {
        float v[GV_MAX_SPLITS];
#pragma unroll
        for (int j = 0; j < GV_MAX_SPLITS; ++j) v[j] = (s0 + j < S) ? coherent_load(p + (size_t)(s0 + j) * stride) : 0.f;
#pragma unroll
        for (int j = 0; j < GV_MAX_SPLITS; ++j)
            if (s0 + j < S) sum += v[j];
    }
    return sum;
}

// Two adjacent columns of sum_splits (64-bit loads), for `np` projections at
// once (pointer p[j], j < np), in groups of G splits: one round trip for up
// to G splits with at most 2 * G * np values in flight.
template <int NP, int G = 8>
__device__ __forceinline__ void sum_splits2(const float* const (&p)[NP], size_t stride, int S, float2 (&out)[NP]) {
#pragma unroll
    for (int j = 0; j < NP; ++j) out[j] = make_float2(0.f, 0.f);
    for (int s0 = 0; s0 < S; s0 += G) {
        float2 v[NP][G];
#pragma unroll
        for (int j = 0; j < NP; ++j)
#pragma unroll
            for (int t = 0; t < G; ++t)
                v[j][t] = (s0 + t < S) ? coherent_load2(p[j] + (size_t)(s0 + t) * stride) : make_float2(0.f, 0.f);
#pragma unroll
        for (int j = 0; j < NP; ++j)
#pragma unroll
            for (int t = 0; t < G; ++t)
                if (s0 + t < S) {
                    out[j].x += v[j][t].x;
                    out[j].y += v[j][t].y;
                }
    }
}

// ------------------------------------------- fixed-point output accumulators
//
// Partial sums of one output element from several workgroups meet in a 64-bit
// accumulator (zero between calls) through atomic adds that return the old
// value; the add that completes the expected count finds the whole sum in the
// returned value, so the hand-off costs one round trip and no separate
// counter.  Integer addition is associative: the result does not depend on
// the order in which contributions arrive.
// Fixed-point format of the accumulators: value * 2^30 + 2^50 per
// contribution in bits 0..57, contribution count in bits 58..63.
constexpr int SK_CNT_SHIFT = 58;
constexpr int SK_MAX_CONTRIB = 63;
constexpr float SK_FX_SCALE = 1073741824.0f;  // 2^30
constexpr float SK_FX_CLAMP = 1048576.0f;     // 2^20: above the fp16 range, so clamped values still give inf
constexpr long long SK_FX_BIAS = 1ll << 50;   // 2^20 * 2^30: keeps every addend non-negative

// One contribution: non-negative addend plus one count.  Non-finite partial
// sums saturate to +-2^20 (NaN to +2^20) and so come out as +-inf.
__device__ __forceinline__ unsigned long long sk_encode(float v) {
    if (!(v == v)) v = SK_FX_CLAMP;
    v = fminf(fmaxf(v, -SK_FX_CLAMP), SK_FX_CLAMP);
    const long long q = (long long)rintf(v * SK_FX_SCALE);  // |q| <= 2^50, exact
    return (unsigned long long)(q + SK_FX_BIAS) + (1ull << SK_CNT_SHIFT);
}

// Value of a completed accumulator holding `cnt` contributions.
__device__ __forceinline__ float sk_decode(unsigned long long total, int cnt) {
    const long long v = (long long)(total & ((1ull << SK_CNT_SHIFT) - 1)) - (long long)cnt * SK_FX_BIAS;
    return (float)v * (1.0f / SK_FX_SCALE);
}

// Two adjacent contributions in flight: the encoded addends and the values
// the atomic adds returned.
struct FxPair {
    unsigned long long ea, eb, oa, ob;
};

// Add a and b to the accumulators acc[0] and acc[1] (device scope).  The
// returned values are only read by fx_finish_pair, so several pairs can be
// in flight before the first wait.
__device__ __forceinline__ FxPair fx_issue_pair(unsigned long long* acc, float a, float b) {
    FxPair f;
    f.ea = sk_encode(a);
    f.eb = sk_encode(b);
    f.oa = __hip_atomic_fetch_add(acc, f.ea, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    f.ob = __hip_atomic_fetch_add(acc + 1, f.eb, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return f;
}

// The add that brought an element to `cnt` contributions stores it to y
// (fp16) and clears the accumulator for the next call.  Both returned values
// are read before any store, and when one add completed both elements (the
// usual case: the last workgroup of a column block completes its pair) the
// two fp16 values go out as one 4-byte store.  Storing the first element
// before reading the second had the wave wait for that store's round trip
// too (config 2 m = 1: 10.97 -> 10.64 us).
// COH: device-coherent stores, for outputs that other workgroups of the same
// launch read.
template <bool COH = false>
__device__ __forceinline__ void fx_finish_pair(const FxPair& f, unsigned long long* acc, int cnt,
                                               EXL3_GLOBAL __half* y) {
    const bool ca = (int)(f.oa >> SK_CNT_SHIFT) == cnt - 1;
    const bool cb = (int)(f.ob >> SK_CNT_SHIFT) == cnt - 1;
    if (!(ca || cb)) return;
    const float va = sk_decode(f.oa + f.ea, cnt), vb = sk_decode(f.ob + f.eb, cnt);
    if (ca && cb) {
        const __half2 v = __floats2half2_rn(va, vb);
        if constexpr (COH)
            __hip_atomic_store(reinterpret_cast<uint32_t*>((__half*)y), *reinterpret_cast<const uint32_t*>(&v),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
            st_h2(y, v);
    } else {
        EXL3_GLOBAL uint16_t* const d = reinterpret_cast<EXL3_GLOBAL uint16_t*>(ca ? y : y + 1);
        const uint16_t h = __half_as_ushort(__float2half_rn(ca ? va : vb));
        if constexpr (COH)
            __hip_atomic_store((uint16_t*)d, h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
            *d = h;
    }
    if (ca) __hip_atomic_store(acc, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (cb) __hip_atomic_store(acc + 1, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void fx_add_pair(unsigned long long* acc, float a, float b, int cnt, EXL3_GLOBAL __half* y) {
    fx_finish_pair(fx_issue_pair(acc, a, b), acc, cnt, y);
}

// Wait until this wave's outstanding memory operations have completed.
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Position (in halves) of the first copy of x'[row][kk] (kk = k offset inside
// the workgroup's range) in the A-fragment staging buffer [m][kts][4][8]:
// quarter Q / slot t of tile row kw = kk % 16 (kw = quarter_row(Q, t)).  Row
// outermost, so a lane's fragments for successive steps and quarters sit at
// compile-time offsets from one base address.
__device__ __forceinline__ int xs_index(int kk, int row, int kts) {
    const int ktl = kk >> 4, kwr = kk & 15;
    const int h = (kwr >> 2) & 1, kp = kwr - 4 * h;
    const int e = (kp & 1) + 2 * ((kp >> 3) & 1) + 4 * ((kp >> 1) & 1);
    const int Q = 2 * h + (e >> 2), t = e & 3;
    return ((row * kts + ktl) * 4 + Q) * 8 + 2 * t;
}

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

template <int K>
__device__ __forceinline__ void load_words(const EXL3_GLOBAL uint32_t* p, uint32_t* w) {
    if constexpr (K == 4 || K == 8) {
#pragma unroll
        for (int h = 0; h < K / 4; ++h) {
            u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const EXL3_GLOBAL u32x4_t*>(p) + h);
            w[4 * h + 0] = v.x; w[4 * h + 1] = v.y; w[4 * h + 2] = v.z; w[4 * h + 3] = v.w;
        }
    } else if constexpr (K == 2) {
        u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const EXL3_GLOBAL u32x2_t*>(p));
        w[0] = v.x; w[1] = v.y;
    } else {
#pragma unroll
        for (int j = 0; j < K; ++j) w[j] = __builtin_nontemporal_load(p + j);
    }
}

// Request the weight words of a wave's first D steps (D: the depth of the
// register ring w).  Loads are unconditional, clamped to the last step, so the
// number in flight is static and each use waits only for its own group.
template <int K, int NS, int D>
__device__ __forceinline__ void prime_weights(uint32_t (&w)[D][K], const EXL3_GLOBAL uint32_t* tb,
                                              size_t step_stride) {
    constexpr int last = NS - 1;
#pragma unroll
    for (int d = 0; d < D; ++d) load_words<K>(tb + (size_t)(d < last ? d : last) * step_stride, w[d]);
}

// One MFMA B fragment (values u = 4F..4F+3 of the lane's group, pair form)
// into every row block's accumulator for its column tile (Q = F / 2, c = F % 2).
template <int K, int CB, int MB, int F>
__device__ __forceinline__ void mv_frag(const uint32_t* buf, const uint32_t* mid, const half8_t (&A)[MB][4],
                                        float4_t (&acc)[MB][2]) {
    uint32_t vf[4];
    vf[0] = decode_pair_word<CB>(window_mid<K, 4 * F + 0>(buf, mid));
    vf[1] = decode_pair_word<CB>(window_mid<K, 4 * F + 1>(buf, mid));
    vf[2] = decode_pair_word<CB>(window_mid<K, 4 * F + 2>(buf, mid));
    vf[3] = decode_pair_word<CB>(window_mid<K, 4 * F + 3>(buf, mid));
    const half8_t B = *reinterpret_cast<const half8_t*>(vf);
    constexpr int Q = F >> 1, c = F & 1;
#pragma unroll
    for (int rb = 0; rb < MB; ++rb) acc[rb][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[rb][Q], B, acc[rb][c], 0, 0, 0);
}

template <int K, int CB, int MB, int... Fs>
__device__ __forceinline__ void mv_frags(const uint32_t* buf, const uint32_t* mid, const half8_t (&A)[MB][4],
                                         float4_t (&acc)[MB][2], std::integer_sequence<int, Fs...>) {
    (mv_frag<K, CB, MB, Fs>(buf, mid, A, acc), ...);
}

// The wave's NS steps: decode 4 k-slices x 2 column tiles per step into MFMA B
// fragments and multiply with the staged activations.  Software-pipelined and
// fully unrolled: each step decodes its words, then reuses their registers to
// request the words of step s + D, so D - 1 groups stay in flight while it
// decodes (D: the depth of the register ring w).  a_base[rb]: this lane's A
// fragments of row block rb in the LDS staging buffer; rows with a_live false
// read nothing and multiply zeros.
template <int K, int CB, int MB, int NS, int D>
__device__ __forceinline__ void decode_mfma_steps(uint32_t (&w)[D][K], const EXL3_GLOBAL uint32_t* tb,
                                                  size_t step_stride, const _Float16* const (&a_base)[MB],
                                                  const bool (&a_live)[MB], float4_t (&acc)[MB][2]) {
    const int lane = threadIdx.x & 63;
    // lane holding the previous group of the same tile (q - 1 mod 8), as a
    // ds_bpermute byte address
    const int prev_addr = ((lane & ~7) | ((lane + 7) & 7)) << 2;
    half8_t A[MB][4];
#pragma unroll
    for (int rb = 0; rb < MB; ++rb)
#pragma unroll
        for (int Q = 0; Q < 4; ++Q) A[rb][Q] = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        const int d = s % D;
        uint32_t buf[K + 1];
#pragma unroll
        for (int j = 0; j < K; ++j) buf[1 + j] = w[d][j];
        buf[0] = (uint32_t)__builtin_amdgcn_ds_bpermute(prev_addr, (int)buf[K]);
#pragma unroll
        for (int rb = 0; rb < MB; ++rb)
            if (a_live[rb]) {
#pragma unroll
                for (int Q = 0; Q < 4; ++Q)
                    A[rb][Q] = *reinterpret_cast<const half8_t*>(a_base[rb] + (s * 16 + Q) * 8);
            }
        uint32_t mid[K];
#pragma unroll
        for (int j = 0; j < K; ++j) mid[j] = __builtin_amdgcn_alignbit(buf[j], buf[j + 1], 16);
        // fragment by fragment (4 words, then its MFMAs), so only one
        // fragment's words are live; each accumulator still takes the
        // quarters Q = 0..3 in order
        mv_frags<K, CB, MB>(buf, mid, A, acc, std::make_integer_sequence<int, 8>{});
        if (s + D < NS) load_words<K>(tb + (size_t)(s + D) * step_stride, w[d]);
    }
}

// GU: the gate/up SwiGLU mode (p.gu), a separate instance so that the plain
// GEMV carries none of its registers (71 against 199 VGPRs at K=4).
template <int K, int CB, int MB, int NS, bool GU, bool XR = false, bool FX = false>
__global__ __launch_bounds__(GV_MAX_THREADS) void gemv_kernel(GemvParams p) {
    constexpr int D = gv_depth<K>();
    extern __shared__ __align__(16) unsigned char gv_smem[];

    const int e = blockIdx.z, bx = blockIdx.x, sidx = blockIdx.y;
    const uint32_t* trellis;
    const __half* suh;
    const __half* svh;
    if (p.t_tab) {
        const int id = gptr(p.ids)[e];
        trellis = reinterpret_cast<const uint32_t*>(gptr(p.t_tab)[id]);
        suh = reinterpret_cast<const __half*>(gptr(p.su_tab)[id]);
        svh = reinterpret_cast<const __half*>(gptr(p.sv_tab)[id]);
    } else if (GU && e) {
        trellis = p.trellis2;
        suh = p.suh2;
        svh = p.svh2;
    } else {
        trellis = p.trellis;
        suh = p.suh;
        svh = p.svh;
    }
    const EXL3_GLOBAL __half* x = gptr(p.x + (long long)e * p.x_stride_e);
    const EXL3_GLOBAL __half* suhg = gptr(suh);
    const int m = p.m, k = p.k, n = p.n, kw = p.kw;
    constexpr int nsteps = NS;
    const int nthreads = 256 * kw, nwaves = 4 * kw;
    const int kts_wg = 4 * nsteps * kw;  // k-slices of this workgroup
    const int ntiles = n >> 4;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int cw = wave & 3, kwi = wave >> 2;
    const int g = lane >> 4, i = lane & 15, q = i & 7;
    const int nt = bx * 8 + cw * 2 + (i >> 3);
    const int kt_wg0 = sidx * kts_wg;
    const int kt_w0 = kt_wg0 + kwi * 4 * nsteps;

    // LDS: x' in A order [m][kts_wg][4][8] halves, zero fragment, per-block
    // sums of x' [m][kts_wg/8] (mul1 correction), partial tiles [kw][m][128]
    const int nblk128 = kts_wg >> 3;
    _Float16* xs = reinterpret_cast<_Float16*>(gv_smem);
    const int xs_halves = kts_wg * 4 * m * 8;
    float* xsum = reinterpret_cast<float*>(gv_smem + (((size_t)xs_halves * 2 + 16 + 15) & ~(size_t)15));
    float* ybuf = xsum + ((m * nblk128 + 3) & ~3);

    // 1. activation loads of this wave's rotation blocks (up to GV_PRE of them),
    //    then every weight load: the activations return first (in-order vmcnt)
    const int nrot = m * nblk128;
    __half2 xpre[GV_PRE], spre[GV_PRE];
#pragma unroll
    for (int j = 0; j < GV_PRE; ++j) {
        const int b = wave + j * nwaves;
        if (b < nrot) {
            const int row = b / nblk128, bb = b - row * nblk128;
            const int kg = kt_wg0 * 16 + bb * 128 + 2 * lane;
            xpre[j] = ld_h2(x + (size_t)row * k + kg);
            if constexpr (!XR) spre[j] = ld_h2(suhg + kg);
        }
    }
    // output scale of this lane's two columns, requested now: the epilogue
    // then needs no extra round trip
    const __half2 svv = ld_h2(gptr(svh) + bx * 128 + 2 * lane);
    uint32_t w[D][K];
    const EXL3_GLOBAL uint32_t* tb = gptr(trellis) + ((size_t)(kt_w0 + g) * ntiles + nt) * (8 * K) + K * q;
    const size_t step_stride = (size_t)4 * ntiles * (8 * K);
    prime_weights<K, NS>(w, tb, step_stride);

    // 2. input rotation of the workgroup's k range into LDS (A order, duplicated)
    if (tid < 8) xs[xs_halves + tid] = (_Float16)0.0f;
    auto rotate = [&](int b, __half2 xv, __half2 sv) {
        const int row = b / nblk128, bb = b - row * nblk128;
        const int kk = bb * 128 + 2 * lane;
        uint32_t bits;
        if constexpr (XR) {
            (void)sv;
            bits = *reinterpret_cast<const uint32_t*>(&xv);
        } else {
            const __half2 pr = __hmul2(xv, sv);
            float a = __low2float(pr), c = __high2float(pr);
            fwht128_pair_fast(a, c, lane);
            const _Float16 ha = f16_rn(a * kHadNorm), hc = f16_rn(c * kHadNorm);
            bits = (uint32_t)__builtin_bit_cast(unsigned short, ha) |
                   ((uint32_t)__builtin_bit_cast(unsigned short, hc) << 16);
        }
        // values kk, kk + 1 sit at xs_index(kk) and + 2 (8-byte aligned):
        // (a, a, c, c) in one 64-bit LDS store
        const uint32_t da = __builtin_amdgcn_perm(bits, bits, 0x01000100u);
        const uint32_t dc = __builtin_amdgcn_perm(bits, bits, 0x03020302u);
        *reinterpret_cast<uint2*>(xs + xs_index(kk, row, kts_wg)) = make_uint2(da, dc);
        if constexpr (CB == 2) {
            const float t = wave_sum(__half2float(__ushort_as_half((unsigned short)(bits & 0xffffu))) +
                                     __half2float(__ushort_as_half((unsigned short)(bits >> 16))));
            if (lane == 0) xsum[b] = t;
        }
    };
#pragma unroll
    for (int j = 0; j < GV_PRE; ++j) {
        const int b = wave + j * nwaves;
        if (b < nrot) rotate(b, xpre[j], spre[j]);
    }
    for (int b = wave + GV_PRE * nwaves; b < nrot; b += nwaves) {
        const int row = b / nblk128, bb = b - row * nblk128;
        const int kg = kt_wg0 * 16 + bb * 128 + 2 * lane;
        rotate(b, ld_h2(x + (size_t)row * k + kg), XR ? __half2{} : ld_h2(suhg + kg));
    }
    __syncthreads();

    // 3. decode + MFMA
    float4_t acc[MB][2];
#pragma unroll
    for (int rb = 0; rb < MB; ++rb) {
        acc[rb][0] = float4_t{0.f, 0.f, 0.f, 0.f};
        acc[rb][1] = float4_t{0.f, 0.f, 0.f, 0.f};
    }
    // A fragments: rows >= m read nothing and keep zeros
    const _Float16* a_base[MB];
    bool a_live[MB];
#pragma unroll
    for (int rb = 0; rb < MB; ++rb) {
        const int row = rb * 16 + i;
        a_live[rb] = row < m;
        a_base[rb] = xs + (size_t)((a_live[rb] ? row : 0) * kts_wg + kwi * 4 * nsteps + g) * 4 * 8;
    }
    decode_mfma_steps<K, CB, MB, NS>(w, tb, step_stride, a_base, a_live, acc);

    // 4. sum the KW k ranges through LDS: ybuf[kwi][m][128], then fold into ybuf[0]
#pragma unroll
    for (int rb = 0; rb < MB; ++rb)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = rb * 16 + 4 * g + r;
                const int col = cw * 32 + (i >> 3) * 16 + (i & 7) + 8 * c;
                if (row < m) ybuf[(kwi * m + row) * 128 + col] = acc[rb][c][r];
            }
    __syncthreads();
    for (int idx = tid; idx < m * 128; idx += nthreads) {
        float v = ybuf[idx];
        for (int j = 1; j < kw; ++j) v += ybuf[j * m * 128 + idx];
        if constexpr (CB == 2) {
            const int row = idx >> 7;
            float sx = 0.f;
            for (int bb = 0; bb < nblk128; ++bb) sx += xsum[row * nblk128 + bb];
            v = v * kMul1Kinv + kMul1Delta * sx;
        }
        ybuf[idx] = v;
    }
    __syncthreads();

    // 5. k-split reduction.
    if constexpr (FX) {
        // one round trip: rotated, scaled partial rows into the fixed-point
        // accumulators; a row's adds are checked after the next row's have
        // been issued, so their round trips overlap
        static_assert(!GU, "one matrix");
        EXL3_GLOBAL __half* yf = gptr(p.y);
        const int c0 = bx * 128 + 2 * lane;
        const float sva = __low2float(svv) * kHadNorm, svb = __high2float(svv) * kHadNorm;
        FxPair fx{};
        int prow = -1;
        for (int row = wave; row < m; row += nwaves) {
            float a = ybuf[row * 128 + 2 * lane], b = ybuf[row * 128 + 2 * lane + 1];
            fwht128_pair_fast(a, b, lane);
            const FxPair cur = fx_issue_pair(p.acc + (size_t)row * n + c0, a * sva, b * svb);
            if (prow >= 0) fx_finish_pair(fx, p.acc + (size_t)prow * n + c0, p.splits, yf + (size_t)prow * n + c0);
            fx = cur;
            prow = row;
        }
        if (prow >= 0) fx_finish_pair(fx, p.acc + (size_t)prow * n + c0, p.splits, yf + (size_t)prow * n + c0);
        return;
    }
    // Otherwise the last workgroup of the column block finishes.  Partials
    // travel through device-coherent (sc1) stores and loads, so the hand-off
    // needs only "my stores completed" before the counter increment; no L2
    // write-back or invalidate.
    const int nblk_n = n >> 7;
    if (p.splits > 1 || GU) {
        const size_t cblk = (size_t)e * nblk_n + bx;
        float* part = p.partials + (cblk * p.splits + sidx) * (size_t)m * 128;
        for (int idx = tid; idx < m * 128; idx += nthreads) coherent_store(part + idx, ybuf[idx]);
        wait_stores();
        __syncthreads();
        __shared__ int is_last;
        // gate/up mode: one counter per column block for both projections
        const size_t ctr = GU ? (size_t)bx : cblk;
        const int arrivals = GU ? 2 * p.splits : p.splits;
        if (tid == 0) {
            const int old = __hip_atomic_fetch_add(p.counters + ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            is_last = (old == arrivals - 1);
        }
        __syncthreads();
        if (!is_last) return;
        if constexpr (GU) {
            // gate and up of each row: split sums (one round trip each), output
            // rotation, norm and svh of both, then the SwiGLU
            if (tid == 0) __hip_atomic_store(p.counters + ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const size_t rstride = (size_t)m * 128;
            const float* pg = p.partials + (size_t)bx * p.splits * rstride;
            const float* pu = p.partials + (size_t)(nblk_n + bx) * p.splits * rstride;
            const int cc = bx * 128 + 2 * lane;
            const __half2 svg = ld_h2(gptr(p.svh) + cc), svu = ld_h2(gptr(p.svh2) + cc);
            const bool clamp = p.limit > 0.0f && p.limit < __builtin_huge_valf();
            EXL3_GLOBAL __half* yg = gptr(p.y);
            for (int row = wave; row < m; row += nwaves) {
                const float* const src[2] = {pg + row * 128 + 2 * lane, pu + row * 128 + 2 * lane};
                float2 gu2[2];
                // groups of 4 splits: 8 splits per group held this instance
                // at 116 VGPRs (4 waves per SIMD) against 68 (7)
                sum_splits2<2, 4>(src, rstride, p.splits, gu2);
                float ga = gu2[0].x, gb = gu2[0].y, ua = gu2[1].x, ub = gu2[1].y;
                fwht128_pair_fast(ga, gb, lane);
                fwht128_pair_fast(ua, ub, lane);
                ga = ga * kHadNorm * __low2float(svg);
                gb = gb * kHadNorm * __high2float(svg);
                ua = ua * kHadNorm * __low2float(svu);
                ub = ub * kHadNorm * __high2float(svu);
                if (clamp) {
                    ga = fminf(ga, p.limit);
                    gb = fminf(gb, p.limit);
                    ua = fminf(fmaxf(ua, -p.limit), p.limit);
                    ub = fminf(fmaxf(ub, -p.limit), p.limit);
                }
                st_h2(yg + (size_t)row * n + cc, h2_rn(silu_f(ga) * ua, silu_f(gb) * ub));
            }
            return;
        }
        const float* base = p.partials + cblk * p.splits * (size_t)m * 128;
        for (int idx = tid; idx < m * 128; idx += nthreads) ybuf[idx] = sum_splits(base + idx, (size_t)m * 128, p.splits);
        if (tid == 0) __hip_atomic_store(p.counters + cblk, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
    }

    // 6. output rotation, svh, fp16 store
    EXL3_GLOBAL __half* y = gptr(p.y + (long long)e * p.y_stride_e);
    const int c0 = bx * 128 + 2 * lane;
    const float sva = __low2float(svv), svb = __high2float(svv);
    for (int row = wave; row < m; row += nwaves) {
        float a = ybuf[row * 128 + 2 * lane], b = ybuf[row * 128 + 2 * lane + 1];
        fwht128_pair_fast(a, b, lane);
        const __half2 o = h2_rn(a * kHadNorm * sva, b * kHadNorm * svb);
        st_h2(y + (size_t)row * n + c0, o);
    }
}

namespace {
// Input rotation of a row batch: xr = fp16( H(x (.) suh) / sqrt(128) ), one
// wave per 128-wide chunk (feeds the k-split GEMV's pre-rotated mode and the
// MFMA GEMM).
// rs (optional): the sum of each chunk's 128 rotated fp16 values, [row][k/128]
// (the mul1 raw-entry GEMM's affine correction).
__global__ __launch_bounds__(256) void rotate_rows_kernel(const __half* x, const __half* suh, __half* xr,
                                                          long long chunks, int k, float* rs = nullptr) {
    const long long chunk = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (chunk >= chunks) return;
    const int lane = threadIdx.x & 63, per_row = k >> 7;
    const long long row = chunk / per_row;
    const int c = (int)(chunk - row * per_row) * 128 + 2 * lane;
    const __half2 pr = __hmul2(ld_h2(gptr(x) + (size_t)row * k + c), ld_h2(gptr(suh) + c));
    float a = __low2float(pr), b = __high2float(pr);
    fwht128_pair_fast(a, b, lane);
    const __half2 o = h2_rn(a * kHadNorm, b * kHadNorm);
    st_h2(gptr(xr) + (size_t)row * k + c, o);
    if (rs) {
        const float t = wave_sum(__low2float(o) + __high2float(o));
        if (lane == 0) gptr(rs)[chunk] = t;
    }
}
}  // namespace

// Dynamic LDS bytes of gemv_kernel for (m, k-slices per workgroup, kw).
inline size_t gemv_smem_bytes(int m, int kts_wg, int kw) {
    const size_t xs = ((size_t)kts_wg * 4 * m * 8 * 2 + 16 + 15) & ~(size_t)15;
    return xs + (size_t)((m * (kts_wg / 8) + 3) & ~3) * 4 + (size_t)kw * m * 128 * 4;
}

template <int K>
int gemv_launch_k(int cb, int mb, const GemvParams& p, int experts, hipStream_t st) {
    dim3 grid(p.n / 128, p.splits, experts);
    const size_t smem = gemv_smem_bytes(p.m, 4 * p.nsteps * p.kw, p.kw);
    const int threads = 256 * p.kw;
#define EXL3_GV_GU(CBV, MBV, NSV, GUV, XRV) EXL3_GV_FX(CBV, MBV, NSV, GUV, XRV, false)
#define EXL3_GV_FX(CBV, MBV, NSV, GUV, XRV, FXV)                                                       \
    if (cb == CBV && mb == MBV && p.nsteps == NSV && (p.gu != 0) == GUV && (p.x_rot != 0) == XRV &&    \
        (p.fx != 0) == FXV) {                                                                          \
        const void* fn = reinterpret_cast<const void*>(&gemv_kernel<K, CBV, MBV, NSV, GUV, XRV, FXV>); \
        const int lrc = allow_dynamic_lds(fn, smem, "exl3 gemv");                                      \
        if (lrc) return lrc;                                                                           \
        gemv_kernel<K, CBV, MBV, NSV, GUV, XRV, FXV><<<grid, threads, smem, st>>>(p);                  \
        return launch_status("exl3 gemv launch");                                                      \
    }
// gate/up mode runs with one row block (m <= 4); pre-rotated rows only in the
// plain mode
// one-round-trip split hand-off for one matrix up to 32 rows (pre-rotated
// rows from 32)
#define EXL3_GV_NS(CBV, MBV, NSV)                                                                      \
    EXL3_GV_GU(CBV, MBV, NSV, false, false) EXL3_GV_GU(CBV, MBV, NSV, false, true)                     \
    if constexpr (MBV == 1) EXL3_GV_GU(CBV, MBV, NSV, true, false)                                     \
    if constexpr (MBV == 1) EXL3_GV_FX(CBV, MBV, NSV, false, false, true)                              \
    if constexpr (MBV == 2) EXL3_GV_FX(CBV, MBV, NSV, false, false, true)                              \
    if constexpr (MBV == 2) EXL3_GV_FX(CBV, MBV, NSV, false, true, true)
#define EXL3_GV_CASE(CBV, MBV) \
    EXL3_GV_NS(CBV, MBV, 2) EXL3_GV_NS(CBV, MBV, 4) EXL3_GV_NS(CBV, MBV, 8) EXL3_GV_NS(CBV, MBV, 16)
    EXL3_GV_CASE(0, 1) EXL3_GV_CASE(0, 2) EXL3_GV_CASE(0, 4)
    EXL3_GV_CASE(1, 1) EXL3_GV_CASE(1, 2) EXL3_GV_CASE(1, 4)
    EXL3_GV_CASE(2, 1) EXL3_GV_CASE(2, 2) EXL3_GV_CASE(2, 4)
#undef EXL3_GV_CASE
#undef EXL3_GV_NS
#undef EXL3_GV_GU
#undef EXL3_GV_FX
    set_error("exl3 gemv: no kernel for codebook %d row blocks %d steps %d", cb, mb, p.nsteps);
    return EXL3_ERR_UNSUPPORTED;
}

// One instantiation unit per K (exl3_gemv_inst.hip built with -DEXL3_K=K).
int gemv_launch(int K, int cb, int mb, const GemvParams& p, int experts, hipStream_t st);

}  // namespace exl3
