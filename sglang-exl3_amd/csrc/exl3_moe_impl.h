// Batched routed-expert MoE layer for gfx950: every active expert of a batch
// of tokens in four launches, with no host synchronisation.
//
//   route    one workgroup groups the (token, slot) entries by expert on the
//            device: active expert list, per-expert row counts/offsets and the
//            compact row -> entry map
//   gate/up  grid (inter/128 column blocks, 2 projections x S k-splits,
//            active-slot capacity): each workgroup is one split of one
//            projection of one expert's column block; the last of its 2S
//            arrivals sums the partials, applies both output rotations,
//            SwiGLU, and the down projection's input rotation of that
//            128-wide chunk, and stores the rotated activation row
//   down     grid (hidden/128, S, slots): same product on the rotated
//            activations; the last arrival applies the output rotation and
//            stores each row at its (token, slot) entry
//   combine  out[t] = sum over slots of w[t,slot] * y[t,slot] in fp32, in slot
//            order (deterministic)
//
// Workgroups of slots beyond the active count exit at once, so the grid is a
// static function of the shapes and the layer can be captured in a HIP graph.
//
// Reference semantics: src/sglang_exl3/exl3.py:520-576 (routed loop: gate/up
// linears, silu(min(g, L)) * clamp(u, -L, L), activation cast to fp16, down
// linear, weighted index_add), exl3.py:960-1110 (batched form with fp16
// gate/up outputs) and csrc/p2b_moe.cu:166-360 (one-token fused kernel).
#pragma once

#include "exl3_gemv_impl.h"

namespace exl3 {

constexpr int MOE_GATE_UP = 0;
constexpr int MOE_DOWN = 1;
constexpr int MOE_ROUTE_THREADS = 1024;

// Device arrays written by moe_route_kernel (inside the caller's workspace).
struct MoeRoute {
    int* num_active;  // [1]
    int* act_expert;  // [slots] expert id of active slot a (ascending ids)
    int* act_off;     // [slots] first compact row of slot a
    int* act_cnt;     // [slots] rows of slot a
    int* rows;        // [entries] compact row -> entry index (token * topk + slot)
};

struct MoeParams {
    MoeRoute rt;
    int topk;
    int entries;       // tokens * topk
    int single_token;  // every entry reads x row 0 (one token)
    const __half* x;   // GATE_UP: tokens [T][k]; DOWN: rotated activations [entries][k] by compact row
    const int64_t* t_tab0;  // projection 0 (gate or down) pointer tables
    const int64_t* su_tab0;
    const int64_t* sv_tab0;
    const int64_t* t_tab1;  // projection 1 (up)
    const int64_t* su_tab1;
    const int64_t* sv_tab1;
    const int64_t* dsu_tab;  // GATE_UP epilogue: the down projection's suh
    float limit;             // SwiGLU clamp; <= 0 or inf: none
    __half* out;             // GATE_UP: [entries][n] by compact row; DOWN: [entries][n] by entry
    float* partials;         // [n/128][nproj][S][entries][128]
    int* counters;           // [slots][n/128]
    int k, n;
    int nproj;      // projections summed by the epilogue (2 gate/up, 1 down)
    int proj_base;  // projection of blockIdx.y / S == 0 in this launch
    int splits;     // S
    int kw;         // k waves per workgroup
    int mode;
};

// ------------------------------------------------------------------ routing

inline size_t moe_route_smem_bytes(int E, int entries) { return (size_t)(3 * E + entries) * sizeof(int); }

// ------------------------------------------------------------ expert GEMVs

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + expf(-g)); }

template <int K, int CB, int MB, int NS>
__global__ __launch_bounds__(GV_MAX_THREADS) void moe_gemv_kernel(MoeParams p) {
    constexpr int ROWS = 16 * MB;
    extern __shared__ __align__(16) unsigned char mv_smem[];

    const int a = blockIdx.z;
    if (a >= gptr(p.rt.num_active)[0]) return;  // slot beyond the active experts
    const int e = gptr(p.rt.act_expert)[a];
    const int roff = gptr(p.rt.act_off)[a];
    const int cnt = gptr(p.rt.act_cnt)[a];
    const int S = p.splits;
    const int pl = blockIdx.y / S, sidx = blockIdx.y - pl * S;
    const int proj = p.proj_base + pl;
    const int bx = blockIdx.x;
    const int64_t* ttab = proj ? p.t_tab1 : p.t_tab0;
    const int64_t* stab = proj ? p.su_tab1 : p.su_tab0;
    const uint32_t* trellis = reinterpret_cast<const uint32_t*>(gptr(ttab)[e]);
    const EXL3_GLOBAL __half* suhg = gptr(reinterpret_cast<const __half*>(gptr(stab)[e]));

    const int k = p.k, n = p.n, kw = p.kw;
    constexpr int nsteps = NS;
    const int nthreads = 256 * kw, nwaves = 4 * kw;
    const int kts_wg = 4 * nsteps * kw;
    const int ntiles = n >> 4;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int cw = wave & 3, kwi = wave >> 2;
    const int g = lane >> 4, i = lane & 15, q = i & 7;
    const int nt = bx * 8 + cw * 2 + (i >> 3);
    const int kt_wg0 = sidx * kts_wg;
    const int kt_w0 = kt_wg0 + kwi * 4 * nsteps;
    const bool pre_rotated = p.mode == MOE_DOWN;

    const int nblk128 = kts_wg >> 3;
    _Float16* xs = reinterpret_cast<_Float16*>(mv_smem);
    const int xs_halves = kts_wg * 4 * ROWS * 8;
    float* xsum = reinterpret_cast<float*>(mv_smem + (((size_t)xs_halves * 2 + 16 + 15) & ~(size_t)15));
    float* ybuf = xsum + ((ROWS * nblk128 + 3) & ~3);
    if (tid < 8) xs[xs_halves + tid] = (_Float16)0.0f;

    const EXL3_GLOBAL uint32_t* tb = gptr(trellis) + ((size_t)(kt_w0 + g) * ntiles + nt) * (8 * K) + K * q;
    const size_t step_stride = (size_t)4 * ntiles * (8 * K);
    const int nblk_n = n >> 7;
    float* part_base = p.partials + ((size_t)(bx * p.nproj + proj) * S + sidx) * (size_t)p.entries * 128;

    for (int r0 = 0; r0 < cnt; r0 += ROWS) {
        const int m = min(ROWS, cnt - r0);
        if (r0 > 0) __syncthreads();  // the previous pass has finished with xs / ybuf

        // source row of activation row `row` of this pass
        auto x_row = [&](int row) -> const EXL3_GLOBAL __half* {
            if (pre_rotated) return gptr(p.x) + (size_t)(roff + r0 + row) * k;
            if (p.single_token) return gptr(p.x);
            const int entry = gptr(p.rt.rows)[roff + r0 + row];
            return gptr(p.x) + (size_t)(entry / p.topk) * k;
        };

        // 1. activation loads (up to GV_PRE blocks per wave), then the weights
        const int nrot = m * nblk128;
        __half2 xpre[GV_PRE], spre[GV_PRE];
#pragma unroll
        for (int j = 0; j < GV_PRE; ++j) {
            const int b = wave + j * nwaves;
            if (b < nrot) {
                const int row = b / nblk128, bb = b - row * nblk128;
                const int kg = kt_wg0 * 16 + bb * 128 + 2 * lane;
                xpre[j] = ld_h2(x_row(row) + kg);
                if (!pre_rotated) spre[j] = ld_h2(suhg + kg);
            }
        }
        uint32_t w[gv_depth<K>()][K];
        prime_weights<K, NS>(w, tb, step_stride);

        // 2. input rotation into the A-order staging buffer (the down
        //    projection's input arrives rotated: staged as is)
        auto stage = [&](int b, __half2 xv, __half2 sv) {
            const int row = b / nblk128, bb = b - row * nblk128;
            const int kk = bb * 128 + 2 * lane;
            _Float16 ha, hc;
            if (pre_rotated) {
                ha = (_Float16)__low2float(xv);
                hc = (_Float16)__high2float(xv);
            } else {
                const __half2 pr = __hmul2(xv, sv);
                float fa = __low2float(pr), fc = __high2float(pr);
                fwht128_pair_f(fa, fc, lane);
                ha = (_Float16)(fa * kHadNorm);
                hc = (_Float16)(fc * kHadNorm);
            }
            const int ia = xs_index(kk, row, kts_wg), ic = xs_index(kk + 1, row, kts_wg);
            xs[ia] = ha;
            xs[ia + 1] = ha;
            xs[ic] = hc;
            xs[ic + 1] = hc;
            if constexpr (CB == 2) {
                float t = (float)ha + (float)hc;
#pragma unroll
                for (int o = 32; o >= 1; o >>= 1) t += __shfl_xor(t, o);
                if (lane == 0) xsum[b] = t;
            }
        };
#pragma unroll
        for (int j = 0; j < GV_PRE; ++j) {
            const int b = wave + j * nwaves;
            if (b < nrot) stage(b, xpre[j], spre[j]);
        }
        for (int b = wave + GV_PRE * nwaves; b < nrot; b += nwaves) {
            const int row = b / nblk128, bb = b - row * nblk128;
            const int kg = kt_wg0 * 16 + bb * 128 + 2 * lane;
            const __half2 sv = pre_rotated ? __half2{} : ld_h2(suhg + kg);
            stage(b, ld_h2(x_row(row) + kg), sv);
        }
        __syncthreads();

        // 3. decode + MFMA
        float4_t acc[MB][2];
#pragma unroll
        for (int rb = 0; rb < MB; ++rb) {
            acc[rb][0] = float4_t{0.f, 0.f, 0.f, 0.f};
            acc[rb][1] = float4_t{0.f, 0.f, 0.f, 0.f};
        }
        const _Float16* a_base[MB];
        bool a_live[MB];
#pragma unroll
        for (int rb = 0; rb < MB; ++rb) {
            const int row = rb * 16 + i;
            a_live[rb] = row < m;
            a_base[rb] = xs + (size_t)((a_live[rb] ? row : 0) * kts_wg + kwi * 4 * nsteps + g) * 4 * 8;
        }
        decode_mfma_steps<K, CB, MB, NS>(w, tb, step_stride, a_base, a_live, acc);

        // 4. k waves summed through LDS, mul1 affine map, partial rows out
#pragma unroll
        for (int rb = 0; rb < MB; ++rb)
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = rb * 16 + 4 * g + r;
                    const int col = cw * 32 + (i >> 3) * 16 + (i & 7) + 8 * c;
                    if (row < m) ybuf[(kwi * ROWS + row) * 128 + col] = acc[rb][c][r];
                }
        __syncthreads();
        for (int idx = tid; idx < m * 128; idx += nthreads) {
            float v = ybuf[idx];
            for (int j = 1; j < kw; ++j) v += ybuf[j * ROWS * 128 + idx];
            if constexpr (CB == 2) {
                const int row = idx >> 7;
                float sx = 0.f;
                for (int bb = 0; bb < nblk128; ++bb) sx += xsum[row * nblk128 + bb];
                v = v * kMul1Kinv + kMul1Delta * sx;
            }
            coherent_store(part_base + (size_t)(roff + r0) * 128 + idx, v);
        }
    }

    // 5. hand-off: the last of nproj * S arrivals for (slot, column block) finishes
    wait_stores();
    __syncthreads();
    __shared__ int is_last;
    const size_t cblk = (size_t)a * nblk_n + bx;
    if (tid == 0) {
        const int total = p.nproj * S;
        const int old = __hip_atomic_fetch_add(p.counters + cblk, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        is_last = (old == total - 1);
    }
    __syncthreads();
    if (!is_last) return;
    if (tid == 0) __hip_atomic_store(p.counters + cblk, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    // 6. epilogue, one row per wave, 2 columns per lane
    const int c0 = bx * 128 + 2 * lane;
    const size_t split_stride = (size_t)p.entries * 128;
    auto sum_proj = [&](int pj, int crow, float& va, float& vb) {
        const float* base = p.partials + (size_t)(bx * p.nproj + pj) * S * split_stride + (size_t)crow * 128 + 2 * lane;
        va = 0.f;
        vb = 0.f;
        for (int s2 = 0; s2 < S; ++s2) {
            va += coherent_load(base + s2 * split_stride);
            vb += coherent_load(base + s2 * split_stride + 1);
        }
    };
    EXL3_GLOBAL __half* outg = gptr(p.out);
    if (p.mode == MOE_GATE_UP) {
        const __half2 gsv = ld_h2(gptr(reinterpret_cast<const __half*>(gptr(p.sv_tab0)[e])) + c0);
        const __half2 usv = ld_h2(gptr(reinterpret_cast<const __half*>(gptr(p.sv_tab1)[e])) + c0);
        const __half2 dsu = ld_h2(gptr(reinterpret_cast<const __half*>(gptr(p.dsu_tab)[e])) + c0);
        const bool clamp = p.limit > 0.0f && p.limit < __builtin_huge_valf();
        for (int row = wave; row < cnt; row += nwaves) {
            const int crow = roff + row;
            float ga, gb, ua, ub;
            sum_proj(0, crow, ga, gb);
            sum_proj(1, crow, ua, ub);
            fwht128_pair_f(ga, gb, lane);
            fwht128_pair_f(ua, ub, lane);
            // gate and up outputs in fp16, as the separate linears return them
            const __half2 gh = __floats2half2_rn(ga * kHadNorm * __low2float(gsv), gb * kHadNorm * __high2float(gsv));
            const __half2 uh = __floats2half2_rn(ua * kHadNorm * __low2float(usv), ub * kHadNorm * __high2float(usv));
            float g0 = __low2float(gh), g1 = __high2float(gh), u0 = __low2float(uh), u1 = __high2float(uh);
            if (clamp) {
                g0 = fminf(g0, p.limit);
                g1 = fminf(g1, p.limit);
                u0 = fminf(fmaxf(u0, -p.limit), p.limit);
                u1 = fminf(fmaxf(u1, -p.limit), p.limit);
            }
            const __half2 act = __floats2half2_rn(silu_f(g0) * u0, silu_f(g1) * u1);
            // input rotation of the down projection for this 128-wide chunk
            const __half2 pr = __hmul2(act, dsu);
            float da = __low2float(pr), db = __high2float(pr);
            fwht128_pair_f(da, db, lane);
            st_h2(outg + (size_t)crow * n + c0, __floats2half2_rn(da * kHadNorm, db * kHadNorm));
        }
    } else {
        const __half2 sv = ld_h2(gptr(reinterpret_cast<const __half*>(gptr(p.sv_tab0)[e])) + c0);
        for (int row = wave; row < cnt; row += nwaves) {
            const int crow = roff + row;
            float va, vb;
            sum_proj(0, crow, va, vb);
            fwht128_pair_f(va, vb, lane);
            const int entry = gptr(p.rt.rows)[crow];
            st_h2(outg + (size_t)entry * n + c0,
                  __floats2half2_rn(va * kHadNorm * __low2float(sv), vb * kHadNorm * __high2float(sv)));
        }
    }
}

// Dynamic LDS bytes of moe_gemv_kernel.
inline size_t moe_smem_bytes(int mb, int kts_wg, int kw) {
    const int rows = 16 * mb;
    const size_t xs = ((size_t)kts_wg * 4 * rows * 8 * 2 + 16 + 15) & ~(size_t)15;
    return xs + (size_t)((rows * (kts_wg / 8) + 3) & ~3) * 4 + (size_t)kw * rows * 128 * 4;
}

template <int K>
int moe_launch_k(int cb, int mb, int ns, const MoeParams& p, dim3 grid, hipStream_t st) {
    const size_t smem = moe_smem_bytes(mb, 4 * ns * p.kw, p.kw);
    const int threads = 256 * p.kw;
#define EXL3_MV_NS(CBV, MBV, NSV)                                                                      \
    if (cb == CBV && mb == MBV && ns == NSV) {                                                         \
        const void* fn = reinterpret_cast<const void*>(&moe_gemv_kernel<K, CBV, MBV, NSV>);            \
        const int lrc = allow_dynamic_lds(fn, smem, "exl3 moe");                                       \
        if (lrc) return lrc;                                                                           \
        moe_gemv_kernel<K, CBV, MBV, NSV><<<grid, threads, smem, st>>>(p);                             \
        return launch_status("exl3 moe launch");                                                      \
    }
#define EXL3_MV_CASE(CBV, MBV) EXL3_MV_NS(CBV, MBV, 2) EXL3_MV_NS(CBV, MBV, 4) EXL3_MV_NS(CBV, MBV, 8)
    EXL3_MV_CASE(0, 1) EXL3_MV_CASE(0, 2) EXL3_MV_CASE(0, 4)
    EXL3_MV_CASE(1, 1) EXL3_MV_CASE(1, 2) EXL3_MV_CASE(1, 4)
    EXL3_MV_CASE(2, 1) EXL3_MV_CASE(2, 2) EXL3_MV_CASE(2, 4)
#undef EXL3_MV_CASE
#undef EXL3_MV_NS
    set_error("exl3 moe: no kernel for codebook %d row blocks %d steps %d", cb, mb, ns);
    return EXL3_ERR_UNSUPPORTED;
}

// One instantiation unit per K (exl3_moe_inst.hip built with -DEXL3_K=K).
int moe_launch(int K, int cb, int mb, int ns, const MoeParams& p, dim3 grid, hipStream_t st);

}  // namespace exl3
