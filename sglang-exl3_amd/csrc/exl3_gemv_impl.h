// Small-m EXL3 GEMV / skinny GEMM kernel for gfx950 (one launch per call).
//
//   y = svh (.) H( x' . T ) / sqrt(128),   x' = fp16( H( fp16(x (.) suh) ) / sqrt(128) )
//
// Reference semantics: csrc/quant/exl3_gemv_kernel.cuh:138-402 (input
// rotation, decode + product, k-split reduce, output rotation).
//
// Layout of the work:
//   grid = (n/128 column blocks, S k-splits, E experts), 256 threads (4 waves).
//   Wave w of a workgroup owns output columns [32w, 32w+32) of its block and
//   walks the block's k-split 4 k-slices (one "step") at a time.  In a step,
//   lane L = 16g + i decodes group q = i%8 of tile (kt0 + g, nt0 + i/8): 32
//   values = MFMA B fragments for columns q and q+8, both k runs, giving four
//   v_mfma_f32_16x16x32_f16 per 16-row block of x.  The MFMA's 32-deep k
//   index (g, e) is the same permutation of tile rows for the A side (x',
//   staged in LDS in that order) and the B side (the decode order), so the
//   contraction is exact whatever order the tile stores k in.
//   All weight loads of the wave are issued before the input-rotation prologue
//   so HBM latency overlaps it.
//   k-split partial sums go to the workspace; the last workgroup of a column
//   block (atomic counter, self-resetting) sums them in split order
//   (deterministic), applies the output FWHT and svh, and stores fp16.
#pragma once

#include "exl3_common.h"
#include "exl3_decode.h"

namespace exl3 {

constexpr int GV_THREADS = 256;

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
    int kts;     // k-slices (16 rows each) per split, multiple of 8
    int splits;  // S
};

// Register budget for the weight words a wave keeps in flight.
template <int K>
__host__ __device__ constexpr int gv_max_steps() {
    return K <= 4 ? 8 : 4;
}

__device__ __forceinline__ void fwht128_pair_f(float& a, float& b, int lane) {
    float s = a + b, d = a - b;
    a = s;
    b = d;
#pragma unroll
    for (int j = 1; j < 64; j <<= 1) {
        float pa = __shfl_xor(a, j), pb = __shfl_xor(b, j);
        if (lane & j) {
            a = pa - a;
            b = pb - b;
        } else {
            a = a + pa;
            b = b + pb;
        }
    }
}

// Device-coherent (sc1) store/load: visible to every workgroup of the device
// without an L2 write-back / invalidate.
__device__ __forceinline__ void coherent_store(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float coherent_load(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until this wave's outstanding memory operations have completed.
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Position (in halves) of x'[row][kk] (kk = k offset inside the split's range)
// in the A-fragment order of the LDS staging buffer [kts][2][m][8].
__device__ __forceinline__ int xs_index(int kk, int row, int m) {
    const int ktl = kk >> 4, kw = kk & 15;
    const int h = (kw >> 2) & 1, kp = kw - 4 * h;
    const int e = (kp & 1) + 2 * ((kp >> 3) & 1) + 4 * ((kp >> 1) & 1);
    return ((ktl * 2 + h) * m + row) * 8 + e;
}

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

template <int K>
__device__ __forceinline__ void load_words(const uint32_t* p, uint32_t* w) {
    if constexpr (K == 4 || K == 8) {
#pragma unroll
        for (int h = 0; h < K / 4; ++h) {
            u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p) + h);
            w[4 * h + 0] = v.x; w[4 * h + 1] = v.y; w[4 * h + 2] = v.z; w[4 * h + 3] = v.w;
        }
    } else if constexpr (K == 2) {
        u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
        w[0] = v.x; w[1] = v.y;
    } else {
#pragma unroll
        for (int j = 0; j < K; ++j) w[j] = __builtin_nontemporal_load(p + j);
    }
}

template <int K, int CB, int MB>
__global__ __launch_bounds__(GV_THREADS) void gemv_kernel(GemvParams p) {
    constexpr int MS = gv_max_steps<K>();
    extern __shared__ __align__(16) unsigned char gv_smem[];

    const int e = blockIdx.z, bx = blockIdx.x, sidx = blockIdx.y;
    const uint32_t* trellis;
    const __half* suh;
    const __half* svh;
    if (p.t_tab) {
        const int id = p.ids[e];
        trellis = reinterpret_cast<const uint32_t*>(p.t_tab[id]);
        suh = reinterpret_cast<const __half*>(p.su_tab[id]);
        svh = reinterpret_cast<const __half*>(p.sv_tab[id]);
    } else {
        trellis = p.trellis;
        suh = p.suh;
        svh = p.svh;
    }
    const __half* x = p.x + (long long)e * p.x_stride_e;
    const int m = p.m, k = p.k, n = p.n, kts = p.kts;
    const int ntiles = n >> 4, nsteps = kts >> 2;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int g = lane >> 4, i = lane & 15, q = i & 7;
    const int nt = bx * 8 + wave * 2 + (i >> 3);
    const int kt0 = sidx * kts;

    // 1. issue every weight load of this wave
    uint32_t w[MS][K];
    {
        const uint32_t* tb = trellis + ((size_t)(kt0 + g) * ntiles + nt) * (8 * K) + K * q;
        const size_t step_stride = (size_t)4 * ntiles * (8 * K);
#pragma unroll
        for (int s = 0; s < MS; ++s)
            if (s < nsteps) load_words<K>(tb + s * step_stride, w[s]);
    }

    // 2. input rotation of this split's k range into LDS (A-fragment order)
    _Float16* xs = reinterpret_cast<_Float16*>(gv_smem);
    const int xs_halves = kts * 2 * m * 8;
    float* ybuf = reinterpret_cast<float*>(gv_smem + ((xs_halves * 2 + 16 + 15) & ~15));
    if (tid < 8) xs[xs_halves + tid] = (_Float16)0.0f;  // zero fragment for rows >= m
    {
        const int nblk = kts >> 3;  // 128-blocks in the split
        for (int b = wave; b < m * nblk; b += GV_THREADS / 64) {
            const int row = b / nblk, bb = b - row * nblk;
            const int kk = bb * 128 + 2 * lane;
            const int kg = kt0 * 16 + kk;
            const __half2 xv = *reinterpret_cast<const __half2*>(x + (size_t)row * k + kg);
            const __half2 sv = *reinterpret_cast<const __half2*>(suh + kg);
            const __half2 pr = __hmul2(xv, sv);
            float a = __low2float(pr), c = __high2float(pr);
            fwht128_pair_f(a, c, lane);
            xs[xs_index(kk, row, m)] = (_Float16)(a * kHadNorm);
            xs[xs_index(kk + 1, row, m)] = (_Float16)(c * kHadNorm);
        }
    }
    __syncthreads();

    // 3. decode + MFMA
    float4_t acc[MB][2];
#pragma unroll
    for (int rb = 0; rb < MB; ++rb) {
        acc[rb][0] = float4_t{0.f, 0.f, 0.f, 0.f};
        acc[rb][1] = float4_t{0.f, 0.f, 0.f, 0.f};
    }
    const int src_lane = (lane & ~7) | ((lane + 7) & 7);
    int a_off[MB];
#pragma unroll
    for (int rb = 0; rb < MB; ++rb) {
        const int row = rb * 16 + i;
        a_off[rb] = row < m ? (g * 2 * m + row) * 8 : -1;
    }
#pragma unroll
    for (int s = 0; s < MS; ++s) {
        if (s < nsteps) {
            uint32_t buf[K + 1];
            buf[0] = __shfl(w[s][K - 1], src_lane);
#pragma unroll
            for (int j = 0; j < K; ++j) buf[1 + j] = w[s][j];
            uint32_t frag[2][2][4];
            decode_group<K, CB, false>(buf, frag);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int rb = 0; rb < MB; ++rb) {
                    const int off = a_off[rb] >= 0 ? a_off[rb] + (s * 4 * 2 * m + h * m) * 8 : xs_halves;
                    const half8_t A = *reinterpret_cast<const half8_t*>(xs + off);
#pragma unroll
                    for (int c = 0; c < 2; ++c) {
                        const half8_t B = *reinterpret_cast<const half8_t*>(frag[c][h]);
                        acc[rb][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, acc[rb][c], 0, 0, 0);
                    }
                }
            }
        }
    }

    // 4. per-block partial tile [m][128] into LDS
#pragma unroll
    for (int rb = 0; rb < MB; ++rb)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = rb * 16 + 4 * g + r;
                const int col = wave * 32 + (i >> 3) * 16 + (i & 7) + 8 * c;
                if (row < m) ybuf[row * 128 + col] = acc[rb][c][r];
            }
    __syncthreads();

    // 5. k-split reduction (last workgroup of the column block finishes).
    // Partials travel through device-coherent (sc1) stores and loads, so the
    // hand-off needs only "my stores completed" before the counter increment;
    // no L2 write-back or invalidate.
    const int nblk_n = n >> 7;
    if (p.splits > 1) {
        const size_t cblk = (size_t)e * nblk_n + bx;
        float* part = p.partials + (cblk * p.splits + sidx) * (size_t)m * 128;
        for (int idx = tid; idx < m * 128; idx += GV_THREADS) coherent_store(part + idx, ybuf[idx]);
        wait_stores();
        __syncthreads();
        __shared__ int is_last;
        if (tid == 0) {
            const int old = __hip_atomic_fetch_add(p.counters + cblk, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            is_last = (old == p.splits - 1);
        }
        __syncthreads();
        if (!is_last) return;
        const float* base = p.partials + cblk * p.splits * (size_t)m * 128;
        for (int idx = tid; idx < m * 128; idx += GV_THREADS) {
            float sum = 0.f;
            for (int s2 = 0; s2 < p.splits; ++s2) sum += coherent_load(base + (size_t)s2 * m * 128 + idx);
            ybuf[idx] = sum;
        }
        if (tid == 0) __hip_atomic_store(p.counters + cblk, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
    }

    // 6. output rotation, svh, fp16 store
    __half* y = p.y + (long long)e * p.y_stride_e;
    const int c0 = bx * 128 + 2 * lane;
    const __half2 svv = *reinterpret_cast<const __half2*>(svh + c0);
    const float sv0 = __low2float(svv), sv1 = __high2float(svv);
    for (int row = wave; row < m; row += GV_THREADS / 64) {
        float a = ybuf[row * 128 + 2 * lane], b = ybuf[row * 128 + 2 * lane + 1];
        fwht128_pair_f(a, b, lane);
        const __half2 o = __floats2half2_rn(a * kHadNorm * sv0, b * kHadNorm * sv1);
        *reinterpret_cast<__half2*>(y + (size_t)row * n + c0) = o;
    }
}

// Dynamic LDS bytes of gemv_kernel for (m, kts).
inline size_t gemv_smem_bytes(int m, int kts) {
    const size_t xs = ((size_t)kts * 2 * m * 8 * 2 + 16 + 15) & ~(size_t)15;
    return xs + (size_t)m * 128 * 4;
}

template <int K>
int gemv_launch_k(int cb, int mb, const GemvParams& p, int experts, hipStream_t st) {
    dim3 grid(p.n / 128, p.splits, experts);
    const size_t smem = gemv_smem_bytes(p.m, p.kts);
#define EXL3_GV_CASE(CBV, MBV)                                                   \
    if (cb == CBV && mb == MBV) {                                                \
        gemv_kernel<K, CBV, MBV><<<grid, GV_THREADS, smem, st>>>(p);             \
        return launch_status("exl3 gemv launch");                                \
    }
    EXL3_GV_CASE(0, 1) EXL3_GV_CASE(0, 2) EXL3_GV_CASE(0, 4)
    EXL3_GV_CASE(1, 1) EXL3_GV_CASE(1, 2) EXL3_GV_CASE(1, 4)
    EXL3_GV_CASE(2, 1) EXL3_GV_CASE(2, 2) EXL3_GV_CASE(2, 4)
#undef EXL3_GV_CASE
    set_error("exl3 gemv: no kernel for codebook %d row blocks %d", cb, mb);
    return EXL3_ERR_UNSUPPORTED;
}

// One instantiation unit per K (exl3_gemv_inst.hip built with -DEXL3_K=K).
int gemv_launch(int K, int cb, int mb, const GemvParams& p, int experts, hipStream_t st);

}  // namespace exl3
