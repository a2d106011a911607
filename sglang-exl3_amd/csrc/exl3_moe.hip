// C ABI of the batched MoE layer (exl3_moe_layer, exl3_p2b_fused_moe) and
// its launch planner.
#include <math.h>
#include <stdlib.h>

#include <mutex>

#include "exl3_fat_impl.h"
#include "exl3_moe_impl.h"

namespace exl3 {

int moe_launch_K1(int, int, const MoeParams&, hipStream_t);
int moe_launch_K2(int, int, const MoeParams&, hipStream_t);
int moe_launch_K3(int, int, const MoeParams&, hipStream_t);
int moe_launch_K4(int, int, const MoeParams&, hipStream_t);
int moe_launch_K5(int, int, const MoeParams&, hipStream_t);
int moe_launch_K6(int, int, const MoeParams&, hipStream_t);
int moe_launch_K7(int, int, const MoeParams&, hipStream_t);
int moe_launch_K8(int, int, const MoeParams&, hipStream_t);

int moe_fused_launch_K1(int, int, int, const MoeParams&, const MoeParams&, hipStream_t);
int moe_fused_launch_K2(int, int, int, const MoeParams&, const MoeParams&, hipStream_t);
int moe_fused_launch_K3(int, int, int, const MoeParams&, const MoeParams&, hipStream_t);
int moe_fused_launch_K4(int, int, int, const MoeParams&, const MoeParams&, hipStream_t);
int moe_fused_launch_K5(int, int, int, const MoeParams&, const MoeParams&, hipStream_t);
int moe_fused_launch_K6(int, int, int, const MoeParams&, const MoeParams&, hipStream_t);
int moe_fused_launch_K7(int, int, int, const MoeParams&, const MoeParams&, hipStream_t);
int moe_fused_launch_K8(int, int, int, const MoeParams&, const MoeParams&, hipStream_t);

int moe_fused_launch(int K, int cb, int nsg, int nsd, const MoeParams& pg, const MoeParams& pd, hipStream_t st) {
    switch (K) {
        case 1: return moe_fused_launch_K1(cb, nsg, nsd, pg, pd, st);
        case 2: return moe_fused_launch_K2(cb, nsg, nsd, pg, pd, st);
        case 3: return moe_fused_launch_K3(cb, nsg, nsd, pg, pd, st);
        case 4: return moe_fused_launch_K4(cb, nsg, nsd, pg, pd, st);
        case 5: return moe_fused_launch_K5(cb, nsg, nsd, pg, pd, st);
        case 6: return moe_fused_launch_K6(cb, nsg, nsd, pg, pd, st);
        case 7: return moe_fused_launch_K7(cb, nsg, nsd, pg, pd, st);
        case 8: return moe_fused_launch_K8(cb, nsg, nsd, pg, pd, st);
    }
    set_error("exl3 moe: K=%d outside 1..8", K);
    return EXL3_ERR_UNSUPPORTED;
}

int moe_launch(int K, int cb, int ns, const MoeParams& p, hipStream_t st) {
    switch (K) {
        case 1: return moe_launch_K1(cb, ns, p, st);
        case 2: return moe_launch_K2(cb, ns, p, st);
        case 3: return moe_launch_K3(cb, ns, p, st);
        case 4: return moe_launch_K4(cb, ns, p, st);
        case 5: return moe_launch_K5(cb, ns, p, st);
        case 6: return moe_launch_K6(cb, ns, p, st);
        case 7: return moe_launch_K7(cb, ns, p, st);
        case 8: return moe_launch_K8(cb, ns, p, st);
    }
    set_error("exl3 moe: K=%d outside 1..8", K);
    return EXL3_ERR_UNSUPPORTED;
}

// ------------------------------------------------------------------ routing

// Group the entries by expert and cut each expert's rows into work units of
// up to 16 rows, with the expert's nine weight addresses resolved.  Entries
// with ids outside [0, E) are dropped.  Row order inside an expert follows
// LDS atomics; each row's product is independent of its position, so results
// do not depend on it.  Also counts each token's valid slots (the fused
// combine's completion count) and, when the combine is fused, writes the zero
// output row of a token without any valid slot.
// (One workgroup of MOE_ROUTE_THREADS threads; rt_smem: moe_route_smem_bytes.)
__device__ __forceinline__ void route_block(int* rt_smem, const int32_t* ids, int entries, int E, MoeTables tabs,
                                            MoeRoute rt, int topk, int* tok_valid, __half* out, int hidden,
                                            int fc) {
    int* cnt = rt_smem;    // [E]
    int* off = cnt + E;    // [E] first compact row
    int* uoff = off + E;   // [E] first unit
    int* pos = uoff + E;   // [entries]
    int* tv = pos + entries;  // [tokens] valid slots
    // Work units are ordered heaviest first: every expert's full 16-row units,
    // then the partial units by row count, descending.  The GEMV kernels take
    // items in that order (in rounds over the grid), so the costly units start
    // first and the cheap ones fill the last round.
    __shared__ int any_empty, rcount[MOE_UNIT_ROWS], rfill[MOE_UNIT_ROWS], rstart[MOE_UNIT_ROWS];
    const int tid = threadIdx.x, tokens = entries / topk;
    for (int e = tid; e < E; e += MOE_ROUTE_THREADS) cnt[e] = 0;
    for (int t = tid; t < tokens; t += MOE_ROUTE_THREADS) tv[t] = 0;
    if (tid < MOE_UNIT_ROWS) {
        rcount[tid] = 0;
        rfill[tid] = 0;
    }
    if (tid == 0) any_empty = 0;
    __syncthreads();
    const EXL3_GLOBAL int32_t* idg = gptr(ids);
    for (int i = tid; i < entries; i += MOE_ROUTE_THREADS) {
        const int e = idg[i];
        const bool valid = e >= 0 && e < E;
        pos[i] = valid ? atomicAdd(&cnt[e], 1) : -1;
        if (valid) atomicAdd(&tv[i / topk], 1);
    }
    __syncthreads();
    for (int t = tid; t < tokens; t += MOE_ROUTE_THREADS) {
        gptr(tok_valid)[t] = tv[t];
        if (tv[t] == 0) any_empty = 1;
    }
    for (int e = tid; e < E; e += MOE_ROUTE_THREADS) {
        const int r = cnt[e] % MOE_UNIT_ROWS;
        if (r) atomicAdd(&rcount[r], 1);
    }
    __syncthreads();
    if (fc && any_empty) {
        const int hp = hidden >> 1;  // fp16 pairs per row
        for (int idx = tid; idx < tokens * hp; idx += MOE_ROUTE_THREADS) {
            const int t = idx / hp;
            if (tv[t] == 0) reinterpret_cast<EXL3_GLOBAL uint32_t*>(gptr(out) + (size_t)t * hidden)[idx - t * hp] = 0u;
        }
    }
    // exclusive scans over the experts (rows, full units, active), one wave
    if (tid < 64) {
        const int chunk = (E + 63) / 64;
        const int e0 = tid * chunk, e1 = min(E, e0 + chunk);
        int sr = 0, su = 0, sa = 0;
        for (int e = e0; e < e1; ++e) {
            const int c = cnt[e];
            sr += c;
            su += c / MOE_UNIT_ROWS;
            sa += c > 0;
        }
        int ir = sr, iu = su, ia = sa;  // inclusive wave scans
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int pr = __shfl_up(ir, d), pu = __shfl_up(iu, d), pa = __shfl_up(ia, d);
            if (tid >= d) {
                ir += pr;
                iu += pu;
                ia += pa;
            }
        }
        int r = ir - sr, uu = iu - su;
        for (int e = e0; e < e1; ++e) {
            off[e] = r;
            uoff[e] = uu;  // first full unit
            r += cnt[e];
            uu += cnt[e] / MOE_UNIT_ROWS;
        }
        if (tid == 63) {
            // partial units after the iu full ones, by row count descending
            int start = iu;
            for (int rr = MOE_UNIT_ROWS - 1; rr >= 1; --rr) {
                rstart[rr] = start;
                start += rcount[rr];
            }
            gptr(rt.counts)[0] = ia;
            gptr(rt.counts)[1] = start;  // work units
            gptr(rt.counts)[2] = ir;     // routed rows
        }
    }
    __syncthreads();
    for (int i = tid; i < entries; i += MOE_ROUTE_THREADS) {
        const int ps = pos[i];
        if (ps >= 0) gptr(rt.rows)[off[idg[i]] + ps] = i;
    }
    for (int e = tid; e < E; e += MOE_ROUTE_THREADS) {
        const int c = cnt[e];
        if (c == 0) continue;
        MoeUnit ud;
        ud.e = e;
        ud.pad = 0;
        ud.pad2 = 0;
#pragma unroll
        for (int j = 0; j < 9; ++j) ud.ptr[j] = reinterpret_cast<const void*>(gptr(tabs.t[j])[e]);
        const int nu = (c + MOE_UNIT_ROWS - 1) / MOE_UNIT_ROWS, nfull = c / MOE_UNIT_ROWS;
        for (int ch = 0; ch < nu; ++ch) {
            ud.nrows = min(MOE_UNIT_ROWS, c - ch * MOE_UNIT_ROWS);
            ud.crow0 = off[e] + ch * MOE_UNIT_ROWS;
            const int slot = ch < nfull ? uoff[e] + ch : rstart[ud.nrows] + atomicAdd(&rfill[ud.nrows], 1);
            const u32x4_t* src = reinterpret_cast<const u32x4_t*>(&ud);
            EXL3_GLOBAL u32x4_t* dst = reinterpret_cast<EXL3_GLOBAL u32x4_t*>(gptr(rt.units) + slot);
#pragma unroll
            for (int j = 0; j < (int)(sizeof(MoeUnit) / 16); ++j) dst[j] = src[j];
        }
    }
}

__global__ __launch_bounds__(MOE_ROUTE_THREADS) void moe_route_kernel(const int32_t* ids, int entries, int E,
                                                                     MoeTables tabs, MoeRoute rt, int topk,
                                                                     int* tok_valid, __half* out, int hidden,
                                                                     int fc) {
    extern __shared__ __align__(16) int rt_smem[];
    route_block(rt_smem, ids, entries, E, tabs, rt, topk, tok_valid, out, hidden, fc);
}

// ------------------------------------------------------------------ rotation

// Input rotation of the gate and up projections, once per (token, slot)
// entry: xr[p][entry] = fp16(FWHT(x[token] (.) suh_p[expert]) / sqrt(128)),
// p = 0 gate, 1 up.  The GEMV items then stage these rows as they are,
// instead of rotating the same rows again for every column block they cover.
// It needs only ids, so it shares a launch with the routing: workgroup 0
// routes, the others rotate, one wave per (entry, projection, 128-block);
// the operations are the GEMV staging's, so the staged values are the same.
__global__ __launch_bounds__(MOE_ROUTE_THREADS) void moe_route_rotate_kernel(
    const int32_t* ids, int entries, int E, MoeTables tabs, MoeRoute rt, int topk, int* tok_valid, __half* out,
    int hidden, int fc, const __half* x, __half* xr) {
    if (blockIdx.x == 0) {
        extern __shared__ __align__(16) int rt_smem[];
        route_block(rt_smem, ids, entries, E, tabs, rt, topk, tok_valid, out, hidden, fc);
        return;
    }
    constexpr int WAVES = MOE_ROUTE_THREADS / 64;
    const int nblk = hidden >> 7, per_entry = 2 * nblk;
    const int job = (blockIdx.x - 1) * WAVES + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int entry = job / per_entry;
    if (entry >= entries) return;
    const int e = gptr(ids)[entry];
    if (e < 0 || e >= E) return;
    const int rem = job - entry * per_entry, proj = rem / nblk, j = rem - proj * nblk;
    const __half* suh = reinterpret_cast<const __half*>(gptr(tabs.t[proj == 0 ? 1 : 4])[e]);
    const int kg = j * 128 + 2 * lane;
    const __half2 pr = __hmul2(ld_h2(gptr(x) + (size_t)(entry / topk) * hidden + kg), ld_h2(gptr(suh) + kg));
    float a = __low2float(pr), c = __high2float(pr);
    fwht128_pair_fast(a, c, lane);
    st_h2(gptr(xr) + ((size_t)proj * entries + entry) * hidden + kg, h2_rn(a * kHadNorm, c * kHadNorm));
}

// ------------------------------------------------------------------ combine

// out[t][c] = fp16( sum_slot w[t][slot] * y[t*topk + slot][c] ), valid slots
// only, fp32 accumulation in slot order.
__global__ __launch_bounds__(256) void moe_combine_kernel(const __half* y, const int32_t* ids, const void* weights,
                                                          int weights_f16, int topk, int E, int hidden,
                                                          __half* out) {
    const int t = blockIdx.y;
    const int c = (blockIdx.x * 256 + threadIdx.x) * 2;
    if (c >= hidden) return;
    float a0 = 0.f, a1 = 0.f;
    for (int s = 0; s < topk; ++s) {
        const int ent = t * topk + s;
        const int id = gptr(ids)[ent];
        if (id < 0 || id >= E) continue;
        const float wv = weights_f16
                             ? __half2float(__ushort_as_half(gptr(reinterpret_cast<const uint16_t*>(weights))[ent]))
                             : gptr(reinterpret_cast<const float*>(weights))[ent];
        const __half2 v = ld_h2(gptr(y) + (size_t)ent * hidden + c);
        a0 += wv * __low2float(v);
        a1 += wv * __high2float(v);
    }
    st_h2(gptr(out) + (size_t)t * hidden + c, h2_rn(a0, a1));
}

static int env_int_once(const char* name) {
    const char* v = getenv(name);
    return (v && *v) ? atoi(v) : 0;
}

int moe_grid_size(const void* fn, int threads, size_t smem) {
    struct Entry {
        const void* fn;
        int threads;
        size_t smem;
        int dev;
        int per_cu, cus;
    };
    static Entry cache[64];
    static int ncache = 0;
    static std::mutex mu;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        set_error("exl3 moe: hipGetDevice failed");
        return -1;
    }
    int per_cu = 0, cus = 0;
    {
        std::lock_guard<std::mutex> lock(mu);
        for (int j = 0; j < ncache && !per_cu; ++j)
            if (cache[j].fn == fn && cache[j].threads == threads && cache[j].smem == smem && cache[j].dev == dev) {
                per_cu = cache[j].per_cu;
                cus = cache[j].cus;
            }
        if (!per_cu) {
            // Workgroups per CU from the kernel's own resources: 4 SIMDs x 512
            // VGPRs (granule 8), at most 8 waves per SIMD, 160 KB of LDS.
            hipFuncAttributes fa;
            if (hipFuncGetAttributes(&fa, fn) != hipSuccess ||
                hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
                set_error("exl3 moe: kernel attribute query failed");
                return -1;
            }
            const int vgprs = ((fa.numRegs > 0 ? fa.numRegs : 128) + 7) & ~7;
            int waves_simd = 512 / vgprs;
            if (waves_simd > 8) waves_simd = 8;
            const int waves_wg = (threads + 63) / 64;
            per_cu = (4 * waves_simd) / waves_wg;
            const size_t lds = smem + fa.sharedSizeBytes;
            if (lds > 0 && (int)(kMaxLds / lds) < per_cu) per_cu = (int)(kMaxLds / lds);
            if (per_cu < 1) per_cu = 1;
            if (cus < 1) cus = 1;
            if (getenv("EXL3_MOE_DEBUG"))
                fprintf(stderr, "exl3 moe grid: regs=%d static_lds=%zu dyn_lds=%zu threads=%d per_cu=%d cus=%d\n",
                        fa.numRegs, (size_t)fa.sharedSizeBytes, smem, threads, per_cu, cus);
            if (ncache < 64) cache[ncache++] = Entry{fn, threads, smem, dev, per_cu, cus};
        }
    }
    const int forced = env_int_once("EXL3_MOE_WG_PER_CU");  // tuning override
    return (forced > 0 ? forced : per_cu) * cus;
}

int moe_fused_grid_size(const void* fn, size_t smem) {
    const int est = moe_grid_size(fn, 256, smem);
    if (est <= 0) return est;
    struct Entry {
        const void* fn;
        size_t smem;
        int dev, resident;
    };
    static Entry cache[32];
    static int ncache = 0;
    static std::mutex mu;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        set_error("exl3 moe: hipGetDevice failed");
        return -1;
    }
    std::lock_guard<std::mutex> lock(mu);
    for (int j = 0; j < ncache; ++j)
        if (cache[j].fn == fn && cache[j].smem == smem && cache[j].dev == dev)
            return est < cache[j].resident ? est : cache[j].resident;
    int cus = 0, nb = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, fn, 256, smem) != hipSuccess || nb < 1 || cus < 1) {
        set_error("exl3 moe: occupancy query failed");
        return -1;
    }
    if (ncache < 32) cache[ncache++] = Entry{fn, smem, dev, nb * cus};
    return est < nb * cus ? est : nb * cus;
}

namespace {

constexpr int kMoeMaxExperts = 4096;
constexpr int kMoeMaxEntries = 8192;

struct MoePlan {
    int ns, kw, splits, bpi;
};

// Active experts expected for `tokens` tokens routed to `topk` of E experts
// uniformly: E (1 - (1 - topk/E)^tokens), capped by the slot count.
double expected_active(int tokens, int topk, int E) {
    const double u = (double)E * (1.0 - pow(1.0 - (double)topk / E, tokens));
    const double cap = (double)(E < tokens * topk ? E : tokens * topk);
    return u < cap ? u : cap;
}

// Launch shape of one expert projection pass, by a rule fitted to graph-timed
// sweeps on MI355X (config 4 at B = 1/16/64 and config 5):
//  * 1 k-wave x 8 steps per workgroup (4 where 32 k-slices do not divide k).
//    With one k-wave the partial rows leave straight from the accumulators, so
//    four workgroups fit a CU; that beat 2 k-waves x 4 steps at every batch
//    (config 4, B = 1 / 16 / 64: 26.2 / 60.1 / 113.9 us against
//    27.0 / 67.5 / 136.7 us);
//  * column blocks per item grouped only when the items would exceed
//    8 x 512 (a few per workgroup of the persistent grid).
// Env overrides (tuning): EXL3_MOE_NSTEPS, EXL3_MOE_KW, EXL3_MOE_BPI.
MoePlan plan_moe(double units, int entries, int k, int n, int nproj, double items12, bool fc_pass = false) {
    (void)entries;
    const int kslices = k / 16, nblk = n / 128;
    const double grid = 512.0;
    int kw = env_int("EXL3_MOE_KW", 1);
    if (kw != 1 && kw != 2) kw = 1;
    // 12-step items (48 k-slices) when k allows and the pass has at least
    // `items12` of them: fewer splits, so fewer hand-offs and partial sums,
    // against fewer items in flight.  With partial-row hand-offs that pays
    // from 1.5 rounds of the ~1024-workgroup grid (down pass, config 4 B = 64:
    // 98.9 -> 92.6 us, config 5 K = 2: 109.1 -> 103.9 us); in the down pass
    // with the fused fixed-point combine every split costs its adds, and it
    // pays from ~700 items (config 4, graph-timed, 4 -> 12 steps: B = 7 / 8 /
    // 12 / 16 with 744 / 816 / 1097 / 1318 items: 34.7 / 37.4 / 41.9 / 45.2 ->
    // 33.4 / 35.2 / 38.4 / 42.2 us; B = 2 / 4 / 6 with 224 / 466 / 657 items:
    // 22.3 / 27.1 / 29.4 -> 24.2 / 28.9 / 30.7 us).
    // With the fused combine (fc_pass) only where they leave one split
    // (k = 768): with two or more the 8-step items win (config 5 down pass,
    // k = 1536: 12 steps and the adds' LDS tile hold two workgroups per CU, 8
    // steps three; K = 2 / 3 / 4 / 5: 101.0 / 110.1 / 108.8 / 123.1 -> 98.8 /
    // 105.8 / 106.5 / 121.3 us).
    int ns = env_int(nproj == 1 ? "EXL3_MOE_DN_NSTEPS" : "EXL3_MOE_GU_NSTEPS", 0);
    if (ns == 0 && kw == 1 && kslices % 48 == 0 && (!fc_pass || kslices == 48) &&
        units * nblk * (kslices / 48) >= items12)
        ns = 12;
    if (ns == 12 && kslices % (4 * ns * kw) == 0 && moe_smem_bytes(4 * ns * kw, kw) <= kMaxLds / 2 - 1024)
        return MoePlan{ns, kw, kslices / (4 * ns * kw), 1};
    if (ns <= 0 || ns == 12) ns = env_int("EXL3_MOE_NSTEPS", 8);
    while (ns > 2 && (kslices % (4 * ns * kw) || (4 * ns * kw) % 8 ||
                      moe_smem_bytes(4 * ns * kw, kw) > kMaxLds / 2 - 1024))
        ns /= 2;
    if (kslices % (4 * ns * kw) || (4 * ns * kw) % 8) {  // k = 128 x odd: 2 steps of 1 wave always divide
        ns = 2;
        kw = 1;
    }
    const int S = kslices / (4 * ns * kw);
    int bpi = env_int("EXL3_MOE_BPI", 0);
    if (bpi <= 0 || nblk % bpi) {
        bpi = 1;
        while (units * (nblk / bpi) * nproj * S > 8.0 * grid) {
            int nb = bpi + 1;
            while (nb <= nblk && nblk % nb) ++nb;
            if (nb > nblk) break;
            bpi = nb;
        }
    }
    return MoePlan{ns, kw, S, bpi};
}

// Batches of at least this many tokens rotate the gate/up input rows once, in
// the routing launch (moe_route_rotate_kernel); a single token (no routing
// launch) has each GEMV item rotate its row.  In the routing launch the
// rotation costs no launch of its own, and it measured faster from two tokens
// on (config 4 B = 2 / 4: 27.9 / 29.4 -> 27.3 / 28.5 us; config 5 K = 2, B = 4:
// 109.0 -> 106.0 us; K = 4: 119.2 -> 115.1 us).
constexpr int kMoeRotTokens = 2;
constexpr int kMoeFusedCombineTokens = 48;
constexpr int kMoeGfxTokens = 3;  // routed batches with the split fixed-point gate/up pass

struct MoeLayout {
    int entries, max_units;
    bool rot, fc;
    bool fr;  // the one-launch gate/up + down pass may run (its own down partials)
    MoePlan gu, dn;
    size_t route_off, units_off, rows_off, tokv_off, h_off, y_off, xr_off, part_off, part_dn_off, total;
};

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

MoeLayout moe_layout(int tokens, int topk, int E, int hidden, int inter) {
    MoeLayout L{};
    L.entries = tokens * topk;
    const int slots = E < L.entries ? E : L.entries;
    L.max_units = slots + (L.entries + MOE_UNIT_ROWS - 1) / MOE_UNIT_ROWS;
    const double act = expected_active(tokens, topk, E);
    const double per = act > 0 ? L.entries / act : 1.0;  // rows per active expert
    const double units = act * ceil(per / MOE_UNIT_ROWS);
    // Up to kMoeFusedCombineTokens tokens the weighted combine runs inside the
    // down pass (fixed-point output accumulators, 8 bytes per output, in the
    // workspace's accumulator region).  Graph-timed on config 4 it saves the
    // combine launch (B = 1 / 2 / 4 / 8 / 16: 27.8 / 32.6 / 36.1 / 49.9 / 64.5 us
    // -> 24.6 / 29.3 / 32.8 / 47.4 / 63.6 us, with 4-step down items).  With
    // 12-step down items (one add per output and slot, no split adds) it pays
    // up to ~48 tokens: B = 17 / 24 / 32 / 48: 51.0 / 51.0 / 59.4 / 72.0 ->
    // 44.0 / 47.7 / 58.4 / 68.2 us; B = 64 even (81.2 / 81.1), B = 96 / 128:
    // 102.4 / 122.0 -> 105.8 / 128.7 us (the contended adds, eight slots per
    // output, cost more than the launch).  Env EXL3_MOE_FC_TOKENS overrides the
    // threshold (0: never fused).
    const int fc_tokens = env_int("EXL3_MOE_FC_TOKENS", kMoeFusedCombineTokens);
    L.fc = tokens <= fc_tokens && (size_t)tokens * hidden * 8 <= kWsAccBytes && topk <= SK_MAX_CONTRIB;
    // the one-launch gate/up + down pass (env EXL3_MOE_FUSED_ROUTED=1) keeps
    // the down items short: 12-step items would hold the launch's LDS (the
    // larger of the two passes') at two workgroups per CU
    L.fr = tokens > 1 && env_int("EXL3_MOE_FUSED_ROUTED", 0) != 0;
    L.gu = plan_moe(units, L.entries, hidden, inter, 2, 1536.0);
    L.dn = plan_moe(units, L.entries, inter, hidden, 1, L.fr ? 1e30 : (L.fc ? 700.0 : 1536.0), L.fc);
    size_t o = kWsScratchOffset;
    L.route_off = o;
    o = align256(o + 4 * sizeof(int));
    L.units_off = o;
    o = align256(o + (size_t)L.max_units * sizeof(MoeUnit));
    L.rows_off = o;
    o = align256(o + (size_t)L.entries * sizeof(int));
    L.tokv_off = o;
    o = align256(o + (size_t)tokens * sizeof(int));
    // h: the rotated activation rows; with the fused combine, room for the
    // fp16 gate and up rows of the split fixed-point gate/up pass instead
    L.h_off = o;
    o = align256(o + (size_t)(L.fc ? 2 : 1) * L.entries * inter * 2);
    L.y_off = o;
    o = align256(o + (size_t)L.entries * hidden * 2);
    L.rot = tokens >= env_int("EXL3_MOE_ROT_TOKENS", kMoeRotTokens);
    L.xr_off = o;
    if (L.rot) o = align256(o + (size_t)2 * L.entries * hidden * 2);
    // split partials: one region that the gate/up and down launches reuse in
    // turn; one token, and routed batches with the one-launch gate/up + down
    // pass (env EXL3_MOE_FUSED_ROUTED=1), get a second one for the down items,
    // which then run alongside the gate/up items
    const bool two = tokens == 1 || L.fr;
    L.part_off = o;
    const size_t pg = (size_t)(inter / 128) * 2 * L.gu.splits;
    const size_t pd = (size_t)(hidden / 128) * 1 * L.dn.splits;
    o = align256(o + (two ? pg : (pg > pd ? pg : pd)) * L.entries * 128 * sizeof(float));
    L.part_dn_off = two ? o : L.part_off;
    if (two) o = align256(o + pd * L.entries * 128 * sizeof(float));
    L.total = o;
    return L;
}

int run_moe_decode(const char* fn, const uint16_t* x, const int32_t* ids, const void* weights, int weights_f16,
                   const MoeTables& tb, int E, uint16_t* out, int tokens, int topk, int hidden, int inter, int KG,
                   int KU, int KD, int cb, float limit, void* ws, size_t ws_bytes, hipStream_t st) {
    EXL3_REQUIRE((long long)tokens * topk <= kMoeMaxEntries, "%s: tokens*topk=%lld above %d", fn,
                 (long long)tokens * topk, kMoeMaxEntries);
    const MoeLayout L = moe_layout(tokens, topk, E, hidden, inter);
    EXL3_REQUIRE_CODE(ws && ws_bytes >= L.total, EXL3_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, %zu given",
                      fn, L.total, ws ? ws_bytes : (size_t)0);
    const int nblk_max = (hidden > inter ? hidden : inter) / 128;
    EXL3_REQUIRE_CODE((size_t)L.max_units * nblk_max <= kWsMaxCounters, EXL3_ERR_UNSUPPORTED,
                      "%s: %d work units x %d column blocks exceed the workspace counters", fn, L.max_units,
                      nblk_max);

    char* w8 = reinterpret_cast<char*>(ws);
    MoeRoute rt;
    rt.counts = reinterpret_cast<int*>(w8 + L.route_off);
    rt.units = reinterpret_cast<MoeUnit*>(w8 + L.units_off);
    rt.rows = reinterpret_cast<int*>(w8 + L.rows_off);
    __half* h = reinterpret_cast<__half*>(w8 + L.h_off);
    __half* yslots = reinterpret_cast<__half*>(w8 + L.y_off);
    int* tok_valid = reinterpret_cast<int*>(w8 + L.tokv_off);

    // One token: every GEMV workgroup maps its unit to a slot of ids itself,
    // and the routing kernel (a launch, ~3 us in a graph) is left out
    const bool direct = tokens == 1 && !L.rot && L.gu.kw == 1 && L.dn.kw == 1 &&
                        (size_t)topk * nblk_max <= kWsMaxCounters && env_int("EXL3_MOE_DIRECT", 1) != 0;

    // 1. routing (with the gate/up input rotation in the same launch for
    //    larger batches)
    __half* xr = reinterpret_cast<__half*>(w8 + L.xr_off);
    if (L.rot) {
        const size_t smem = moe_route_smem_bytes(E, L.entries, tokens);
        int rc = allow_dynamic_lds(reinterpret_cast<const void*>(&moe_route_rotate_kernel), smem,
                                   "exl3 moe route+rotate");
        if (rc) return rc;
        const long long jobs = (long long)L.entries * 2 * (hidden / 128);
        const long long blocks = 1 + (jobs + MOE_ROUTE_THREADS / 64 - 1) / (MOE_ROUTE_THREADS / 64);
        moe_route_rotate_kernel<<<(unsigned)blocks, MOE_ROUTE_THREADS, smem, st>>>(
            ids, L.entries, E, tb, rt, topk, tok_valid, reinterpret_cast<__half*>(out), hidden, L.fc,
            reinterpret_cast<const __half*>(x), xr);
        rc = launch_status("exl3 moe route+rotate launch");
        if (rc) return rc;
    } else if (!direct) {
        const size_t smem = moe_route_smem_bytes(E, L.entries, tokens);
        int rc = allow_dynamic_lds(reinterpret_cast<const void*>(&moe_route_kernel), smem, "exl3 moe route");
        if (rc) return rc;
        moe_route_kernel<<<1, MOE_ROUTE_THREADS, smem, st>>>(ids, L.entries, E, tb, rt, topk, tok_valid,
                                                             reinterpret_cast<__half*>(out), hidden, L.fc);
        rc = launch_status("exl3 moe route launch");
        if (rc) return rc;
    }

    MoeParams p{};
    p.rt = rt;
    p.topk = topk;
    p.entries = L.entries;
    p.single_token = tokens == 1;
    p.limit = limit;
    p.counters = reinterpret_cast<int*>(w8);
    p.partials = reinterpret_cast<float*>(w8 + L.part_off);
    p.direct = direct;
    p.tab_prefetch = env_int("EXL3_MOE_TAB_PREFETCH", 1) != 0;
    // routed passes pick their column blocks per item from the unit count
    // (moe_item_bpi); env EXL3_MOE_BPI forces the planner's value, and
    // EXL3_MOE_BPI_DYN=0 keeps it
    p.bpi_dyn = env_int("EXL3_MOE_BPI", 0) <= 0 && env_int("EXL3_MOE_BPI_DYN", 1) != 0;
    p.ids = ids;
    p.E = E;
    p.tabs = tb;

    // One token, one K for all three projections: gate/up and down can run
    // in one persistent launch (moe_fused_direct_kernel), opt-in with env
    // EXL3_MOE_FUSED=1.  It gives the same bits but is not the default:
    // graph-timed on config 4 (layers back to back) the fused kernel takes
    // 22.4 us against 11.6 + 9.8 us for the two launches, whose boundary
    // costs ~0.3 us; the down items, started early, decode more slowly next
    // to the running gate/up items than the down launch does alone.
    // readiness flag rows 1 KB apart: the polls of one unit's down items
    // stay off the lines of other units' flags and of the hand-off counters
    int ready_stride = env_int("EXL3_MOE_READY_STRIDE", 256);
    if (ready_stride < inter / 128) ready_stride = inter / 128;
    const bool fuse_req = direct && KG == KU && KU == KD && L.gu.kw == 1 && L.dn.kw == 1 &&
                          moe_fused_steps_ok(L.dn.ns) &&
                          (size_t)topk * (inter / 128 + hidden / 128 + ready_stride + 1) + 258 <= kWsMaxCounters &&
                          env_int("EXL3_MOE_FUSED", 0) != 0;

    // the fused combine one round trip per split (each split adds its rotated
    // partial rows into the output accumulators) when every token's count of
    // contributions (valid slots x splits) fits the accumulators' count bits
    const bool dn_fxs = L.fc && L.dn.kw == 1 && topk * L.dn.splits <= SK_MAX_CONTRIB && env_int("EXL3_MOE_FXS", 1) != 0;
    // Gate/up by split fixed-point adds (no partial rows, counter or last
    // arrival; each element's completing add writes the fp16 gate or up
    // value), and the down pass stages the SwiGLU from those rows, rotated with
    // its own suh.  The split hand-off being one round trip, the gate/up items
    // are cut finer for one token (env EXL3_MOE_GFX_GU_NSTEPS; default 4 steps
    // there, the planner's otherwise).  One token (direct) or rotated routed
    // batches up to kMoeGfxTokens (env EXL3_MOE_GFX_TOKENS; EXL3_MOE_GFX=0
    // keeps the partial-row hand-off).  Graph-timed on config 4, partial rows
    // -> split fixed-point: B = 1 / 2 / 3: 19.0 / 24.2 / 25.8 -> 16.8 / 22.6 /
    // 24.1 us; B = 4 / 6: 27.9 / 29.9 -> 28.8 / 31.1; B = 8 / 12: 38.9 / 43.2
    // -> 37.0 / 41.7; B = 16: 47.1 -> 49.2 (16-row units: every down item
    // then rotates up to 16 SwiGLU rows per k block, and the adds contend).
    const int gu_kslices = hidden / 16;
    const int gfx_ns = env_int("EXL3_MOE_GFX_GU_NSTEPS", direct ? (fuse_req ? 8 : 4) : L.gu.ns);
    // With 8 or more gate/up splits the partial-row hand-off's last arrival
    // reads 2 S >= 16 partial rows per element, and the split fixed-point
    // pass pays one token further (config 5, 4 tokens, 8 splits, K = 2 / 3 /
    // 4 / 5: 99.0 / 106.2 / 107.8 / 121.8 -> 95.4 / 100.3 / 101.3 / 117.2 us;
    // config 4, 4 splits, Zipf router, B = 4 / 5 / 6: 27.4 / 30.0 / 29.1 ->
    // 29.2 / 30.8 / 31.1 us with it).
    const int gfx_tokens = env_int("EXL3_MOE_GFX_TOKENS", kMoeGfxTokens +
                                                          (gu_kslices % (4 * gfx_ns) == 0 && gu_kslices / (4 * gfx_ns) >= 8));
    const bool gfx = (direct || (L.rot && tokens <= gfx_tokens)) &&
                     dn_fxs && moe_gfx_steps_ok(gfx_ns) && moe_gfx_steps_ok(L.dn.ns) &&
                     gu_kslices % (4 * gfx_ns) == 0 && gu_kslices / (4 * gfx_ns) <= SK_MAX_CONTRIB &&
                     ((size_t)tokens * hidden + (size_t)2 * L.entries * inter) * 8 <= kWsAccBytes &&
                     env_int("EXL3_MOE_GFX", 1) != 0;
    const int gu_ns = gfx ? gfx_ns : L.gu.ns;
    const bool fused = fuse_req && moe_fused_steps_ok(gu_ns);
    // Routed batch, gate/up and down in one launch after the routing launch
    // (moe_fused_routed_kernel; opt-in, env EXL3_MOE_FUSED_ROUTED=1): counters
    // [gate/up hand-off | down hand-off | readiness counts | done counts] per
    // work unit in the zeroed counter region
    const size_t fr_units = (size_t)L.max_units;
    const size_t fr_ready = (fr_units * (inter / 128 + hidden / 128) + 255) & ~(size_t)255;
    const bool fused_routed = L.fr && !direct && L.rot && KG == KU && KU == KD && L.gu.kw == 1 && L.dn.kw == 1 &&
                              moe_fused_routed_steps_ok(gu_ns, L.dn.ns, gfx, dn_fxs) &&
                              fr_ready + fr_units * (ready_stride + 1) <= kWsMaxCounters;
    unsigned long long* const acc_base = reinterpret_cast<unsigned long long*>(w8 + kWsAccOffset);

    // 3. gate + up (+ SwiGLU + down input rotation; GFX: the gate and up rows)
    p.mode = MOE_GATE_UP;
    p.x = L.rot ? xr : reinterpret_cast<const __half*>(x);
    p.in_rot = L.rot;
    p.out = h;
    p.k = hidden;
    p.n = inter;
    p.nproj = 2;
    p.splits = gfx ? gu_kslices / (4 * gfx_ns) : L.gu.splits;
    p.gfx = gfx;
    p.fxs = gfx;
    if (gfx) p.acc = acc_base + (size_t)tokens * hidden;  // [2][entries][inter], after the output's
    p.kw = L.gu.kw;
    p.bx_per_item = L.gu.bpi;
    int rc;
    MoeParams pg = p;  // the gate/up pass, kept for the fused launch
    pg.proj_base = 0;
    pg.proj_launch = 2;
    if (fused) {
        // counters: [gate/up hand-off | down hand-off | readiness flags | done
        // counts | item ticket, finished workgroups]
        const int nbg = inter / 128, nbd = hidden / 128;
        int* c0 = reinterpret_cast<int*>(w8);
        pg.ready = c0 + (((size_t)topk * (nbg + nbd) + 255) & ~(size_t)255);
        pg.done = pg.ready + (size_t)topk * ready_stride;
        pg.ticket = pg.done + topk;
        pg.max_polls = wait_polls();
        pg.status = c0 + kWsStatusIndex;
        pg.ready_nblk = nbg;
        pg.ready_stride = ready_stride;
        pg.ready_target = gfx ? 2 * pg.splits : 1;
        pg.poll_sleep = env_int("EXL3_MOE_POLL_SLEEP", 1);
        pg.prime_late = env_int("EXL3_MOE_PRIME_LATE", 0);
    } else if (fused_routed) {
        int* c0 = reinterpret_cast<int*>(w8);
        pg.ready = c0 + fr_ready;
        pg.done = pg.ready + fr_units * ready_stride;
        pg.ticket = nullptr;
        pg.max_polls = wait_polls();
        pg.status = c0 + kWsStatusIndex;
        pg.ready_nblk = inter / 128;
        pg.ready_stride = ready_stride;
        pg.ready_target = gfx ? 2 * pg.splits : 1;
        pg.poll_sleep = env_int("EXL3_MOE_POLL_SLEEP", 1);
        pg.prime_late = env_int("EXL3_MOE_PRIME_LATE", 0);
    } else if (KG == KU) {
        p.proj_base = 0;
        p.proj_launch = 2;
        rc = moe_launch(KG, cb, gu_ns, p, st);
        if (rc) return rc;
    } else {
        p.proj_launch = 1;
        p.proj_base = 0;
        rc = moe_launch(KG, cb, gu_ns, p, st);
        if (rc) return rc;
        p.proj_base = 1;
        rc = moe_launch(KU, cb, gu_ns, p, st);
        if (rc) return rc;
    }

    // 4. down
    p.mode = MOE_DOWN;
    p.in_rot = 0;
    p.x = h;
    p.out = yslots;
    p.k = inter;
    p.n = hidden;
    p.nproj = 1;
    p.proj_base = 0;
    p.proj_launch = 1;
    p.splits = L.dn.splits;
    p.kw = L.dn.kw;
    p.bx_per_item = L.dn.bpi;
    p.fc = L.fc;
    p.acc = acc_base;
    p.tok_valid = tok_valid;
    p.weights = weights;
    p.weights_f16 = weights_f16;
    p.final_out = reinterpret_cast<__half*>(out);
    p.fxs = dn_fxs;
    if (fused || fused_routed) {
        p.counters = reinterpret_cast<int*>(w8) + (fused ? (size_t)topk : fr_units) * (inter / 128);
        p.partials = reinterpret_cast<float*>(w8 + L.part_dn_off);
        p.ready = pg.ready;
        p.done = pg.done;
        p.ready_nblk = pg.ready_nblk;
        p.ready_stride = pg.ready_stride;
        p.ready_target = pg.ready_target;
        p.poll_sleep = pg.poll_sleep;
        p.prime_late = pg.prime_late;
        p.max_polls = pg.max_polls;
        p.status = pg.status;
        p.ticket = pg.ticket;
        p.dn_items_per_unit = ((hidden / 128) / L.dn.bpi) * L.dn.splits;
        p.gfx = gfx;
        rc = moe_fused_launch(KD, cb, gu_ns, L.dn.ns, pg, p, st);
    } else {
        rc = moe_launch(KD, cb, L.dn.ns, p, st);
    }
    if (rc) return rc;
    if (L.fc) return EXL3_OK;

    // 5. weighted combine
    moe_combine_kernel<<<dim3((hidden / 2 + 255) / 256, tokens), 256, 0, st>>>(
        yslots, ids, weights, weights_f16, topk, E, hidden, reinterpret_cast<__half*>(out));
    return launch_status("exl3 moe combine launch");
}

// ------------------------------------------------------------ prefill path
//
// For batches whose experts get many rows each, the 16-row work units of the
// decode path decode every expert's weights once per 16 rows with the
// pair-form GEMV.  The prefill path groups the rows of each expert into tiles
// of up to 64 / 128 rows and runs the MFMA GEMM kernel (real-valued B
// fragments, decode once per tile) in its grouped mode:
//   route    one workgroup: counting sort of the (token, slot) entries by
//            expert -> compact row -> entry map, row tiles (expert, first row,
//            rows), the tile count
//   rotate   xr[p][crow] = fp16(H(x[token] (.) suh_p[e]) / sqrt(128)) for the
//            gate and up projections, one wave per (row, projection, block)
//   gate     g32[crow] = fp32 gate output
//   up       h[crow] = fp16 silu(min(g, L)) * clamp(u, -L, L), rotated with the
//            down projection's suh
//   down     y[entry] = fp16 down output
//   combine  out[t] = sum over the token's valid slots of w * y, fp32, slot order
// Every grid is a function of the shapes only (tiles past the device count
// exit at once), so the layer stays capturable in a HIP graph; batches above
// kMoePrefillChunk entries run as consecutive token chunks.  The reference
// runs these experts through a host loop over experts (counts.tolist()) into
// exl3_fat_gemm / exl3_fat_gemm_scatter (src/sglang_exl3/exl3.py:1154-1231,
// 1234-1344).
constexpr int kMoePrefillChunk = 16384;  // (token, slot) entries per pipeline pass

__global__ __launch_bounds__(MOE_ROUTE_THREADS) void moe_prefill_route_kernel(const int32_t* ids, int entries,
                                                                             int E, int mt, int* pos, int* rows,
                                                                             FatTile* tiles, int* counts) {
    extern __shared__ __align__(16) int prs[];
    int* cnt = prs;       // [E]
    int* off = cnt + E;   // [E] first compact row
    int* toff = off + E;  // [E] first tile
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += MOE_ROUTE_THREADS) cnt[e] = 0;
    __syncthreads();
    const EXL3_GLOBAL int32_t* idg = gptr(ids);
    EXL3_GLOBAL int* posg = gptr(pos);
    for (int i = tid; i < entries; i += MOE_ROUTE_THREADS) {
        const int e = idg[i];
        posg[i] = (e >= 0 && e < E) ? atomicAdd(&cnt[e], 1) : -1;
    }
    __syncthreads();
    if (tid < 64) {  // exclusive scans of rows and tiles over the experts, one wave
        const int chunk = (E + 63) / 64;
        const int e0 = tid * chunk, e1 = min(E, e0 + chunk);
        int sr = 0, st = 0;
        for (int e = e0; e < e1; ++e) {
            sr += cnt[e];
            st += (cnt[e] + mt - 1) / mt;
        }
        int ir = sr, it = st;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int pr = __shfl_up(ir, d), pt = __shfl_up(it, d);
            if (tid >= d) {
                ir += pr;
                it += pt;
            }
        }
        int r = ir - sr, t = it - st;
        for (int e = e0; e < e1; ++e) {
            off[e] = r;
            toff[e] = t;
            r += cnt[e];
            t += (cnt[e] + mt - 1) / mt;
        }
        if (tid == 63) {
            gptr(counts)[0] = it;  // row tiles
            gptr(counts)[1] = ir;  // routed rows
        }
    }
    __syncthreads();
    for (int i = tid; i < entries; i += MOE_ROUTE_THREADS) {  // the same i as above: own pos[] write
        const int ps = posg[i];
        if (ps >= 0) gptr(rows)[off[idg[i]] + ps] = i;
    }
    for (int e = tid; e < E; e += MOE_ROUTE_THREADS) {
        const int c = cnt[e];
        for (int t = 0; t * mt < c; ++t) {
            FatTile tl;
            tl.e = e;
            tl.crow0 = off[e] + t * mt;
            tl.nrows = min(mt, c - t * mt);
            tl.pad = 0;
            *reinterpret_cast<EXL3_GLOBAL u32x4_t*>(gptr(tiles) + toff[e] + t) = *reinterpret_cast<const u32x4_t*>(&tl);
        }
    }
}

// xr[p][crow][k] = fp16(FWHT(x[token][k] (.) suh_p[e][k]) / sqrt(128)), p = 0 gate, 1 up; one wave per
// (compact row, projection) walking the row's 128-wide blocks (the loads of the next block are issued
// before the current block's transform); rows past the routed count exit.
__global__ __launch_bounds__(256) void moe_prefill_rotate_kernel(const __half* x, const int32_t* ids, const int* rows,
                                                                const int* counts, const int64_t* suh_g,
                                                                const int64_t* suh_u, int topk, int hidden,
                                                                int entries, __half* xr) {
    const int nblk = hidden >> 7;
    const int job = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int crow = job >> 1, proj = job & 1;
    if (crow >= gptr(counts)[1]) return;
    const int entry = gptr(rows)[crow];
    const int e = gptr(ids)[entry];
    const EXL3_GLOBAL __half* suh = gptr(reinterpret_cast<const __half*>(gptr(proj ? suh_u : suh_g)[e])) + 2 * lane;
    const EXL3_GLOBAL __half* xs = gptr(x) + (size_t)(entry / topk) * hidden + 2 * lane;
    EXL3_GLOBAL __half* dst = gptr(xr) + ((size_t)proj * entries + crow) * hidden + 2 * lane;
    __half2 xv = ld_h2(xs), sv = ld_h2(suh);
    for (int j = 0; j < nblk; ++j) {
        const __half2 pr = __hmul2(xv, sv);
        if (j + 1 < nblk) {
            xv = ld_h2(xs + (j + 1) * 128);
            sv = ld_h2(suh + (j + 1) * 128);
        }
        float a = __low2float(pr), c = __high2float(pr);
        fwht128_pair_fast(a, c, lane);
        st_h2(dst + j * 128, h2_rn(a * kHadNorm, c * kHadNorm));
    }
}

struct PrefillLayout {
    int chunk_tokens, entries, mt, max_tiles;
    size_t counts_off, pos_off, rows_off, tiles_off, xr_off, g_off, h_off, y_off, total;
};

PrefillLayout prefill_layout(int tokens, int topk, int E, int hidden, int inter) {
    PrefillLayout L{};
    L.chunk_tokens = kMoePrefillChunk / topk < 1 ? 1 : kMoePrefillChunk / topk;
    if (L.chunk_tokens > tokens) L.chunk_tokens = tokens;
    L.entries = L.chunk_tokens * topk;
    // 64-row tiles: the 128-row variant holds 67 KB of LDS, so only two
    // workgroups share a CU, and measured slower per row (config 4, 2048
    // tokens: 311 us per grouped GEMM launch against 2 x 120 us at 64 rows)
    L.mt = 64;
    L.max_tiles = (E < L.entries ? E : L.entries) + L.entries / L.mt;
    size_t o = kWsScratchOffset;
    L.counts_off = o;
    o = align256(o + 4 * sizeof(int));
    L.pos_off = o;
    o = align256(o + (size_t)L.entries * sizeof(int));
    L.rows_off = o;
    o = align256(o + (size_t)L.entries * sizeof(int));
    L.tiles_off = o;
    o = align256(o + (size_t)L.max_tiles * sizeof(FatTile));
    L.xr_off = o;
    o = align256(o + (size_t)2 * L.entries * hidden * 2);
    L.g_off = o;
    o = align256(o + (size_t)L.entries * inter * 4);
    L.h_off = o;
    o = align256(o + (size_t)L.entries * inter * 2);
    L.y_off = o;
    o = align256(o + (size_t)L.entries * hidden * 2);
    L.total = o;
    return L;
}

// Rows per active expert (uniform routing estimate) from which a batch takes
// the prefill path; every batch above the decode path's entry limit does.
// Graph-timed on config 4 (decode path -> prefill path): B = 64 / 128: 92 /
// 151 us -> 135 / 158 us; B = 256 / 512 / 1024: 243 / 398 / 772 us -> 217 /
// 298 / 437 us.
constexpr double kMoePrefillRowsPerExpert = 16.0;

bool moe_use_prefill(int tokens, int topk, int E) {
    const int forced = env_int("EXL3_MOE_PREFILL", -1);  // 0: never (decode path), 1: always
    const long long entries = (long long)tokens * topk;
    if (entries > kMoeMaxEntries) return true;
    if (forced >= 0) return forced != 0;
    const double act = expected_active(tokens, topk, E);
    return act > 0 && (double)entries / act >= kMoePrefillRowsPerExpert;
}

int run_moe_prefill(const char* fn, const uint16_t* x, const int32_t* ids, const void* weights, int weights_f16,
                    const MoeTables& tb, int E, uint16_t* out, int tokens, int topk, int hidden, int inter, int KG,
                    int KU, int KD, int cb, float limit, void* ws, size_t ws_bytes, hipStream_t st) {
    const PrefillLayout L = prefill_layout(tokens, topk, E, hidden, inter);
    EXL3_REQUIRE_CODE(ws && ws_bytes >= L.total, EXL3_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, %zu given",
                      fn, L.total, ws ? ws_bytes : (size_t)0);
    char* w8 = reinterpret_cast<char*>(ws);
    int* counts = reinterpret_cast<int*>(w8 + L.counts_off);
    int* pos = reinterpret_cast<int*>(w8 + L.pos_off);
    int* rows = reinterpret_cast<int*>(w8 + L.rows_off);
    FatTile* tiles = reinterpret_cast<FatTile*>(w8 + L.tiles_off);
    __half* xr = reinterpret_cast<__half*>(w8 + L.xr_off);
    float* g32 = reinterpret_cast<float*>(w8 + L.g_off);
    __half* h = reinterpret_cast<__half*>(w8 + L.h_off);
    __half* y = reinterpret_cast<__half*>(w8 + L.y_off);
    const size_t rsmem = (size_t)3 * E * sizeof(int);
    int rc = allow_dynamic_lds(reinterpret_cast<const void*>(&moe_prefill_route_kernel), rsmem, "exl3 moe prefill route");
    if (rc) return rc;
    const size_t wsz = weights_f16 ? 2 : 4;
    for (int t0 = 0; t0 < tokens; t0 += L.chunk_tokens) {
        const int T = tokens - t0 < L.chunk_tokens ? tokens - t0 : L.chunk_tokens;
        const int entries = T * topk;
        const int32_t* idc = ids + (size_t)t0 * topk;
        moe_prefill_route_kernel<<<1, MOE_ROUTE_THREADS, rsmem, st>>>(idc, entries, E, L.mt, pos, rows, tiles,
                                                                       counts);
        rc = launch_status("exl3 moe prefill route launch");
        if (rc) return rc;
        const long long jobs = (long long)entries * 2;
        moe_prefill_rotate_kernel<<<(unsigned)((jobs + 3) / 4), 256, 0, st>>>(
            reinterpret_cast<const __half*>(x) + (size_t)t0 * hidden, idc, rows, counts, tb.t[1], tb.t[4], topk,
            hidden, entries, xr);
        rc = launch_status("exl3 moe prefill rotate launch");
        if (rc) return rc;
        FatParams p{};
        p.M = L.max_tiles * L.mt;  // grid.y = max_tiles; rows come from the tiles
        p.tiles = tiles;
        p.ntiles = counts;
        for (int j = 0; j < 9; ++j) p.tabs[j] = tb.t[j];
        p.g32 = g32;
        p.rows_map = rows;
        p.limit = limit;
        // gate
        p.gmode = 1;
        p.a = xr;
        p.k = hidden;
        p.n = inter;
        p.ksteps = hidden / 64;
        rc = fat_launch(KG, cb, L.mt, p, 1, st);
        if (rc) return rc;
        // up, with the SwiGLU and the down projection's input rotation
        p.gmode = 2;
        p.a = xr + (size_t)entries * hidden;
        p.out16 = h;
        rc = fat_launch(KU, cb, L.mt, p, 1, st);
        if (rc) return rc;
        // down, by (token, slot) entry
        p.gmode = 3;
        p.a = h;
        p.k = inter;
        p.n = hidden;
        p.ksteps = inter / 64;
        p.out16 = y;
        rc = fat_launch(KD, cb, L.mt, p, 1, st);
        if (rc) return rc;
        moe_combine_kernel<<<dim3((hidden / 2 + 255) / 256, T), 256, 0, st>>>(
            y, idc, reinterpret_cast<const char*>(weights) + (size_t)t0 * topk * wsz, weights_f16, topk, E, hidden,
            reinterpret_cast<__half*>(out) + (size_t)t0 * hidden);
        rc = launch_status("exl3 moe prefill combine launch");
        if (rc) return rc;
    }
    return EXL3_OK;
}

int run_moe(const char* fn, const uint16_t* x, const int32_t* ids, const void* weights, int weights_f16,
            const MoeTables& tb, int E, uint16_t* out, int tokens, int topk, int hidden, int inter, int KG,
            int KU, int KD, int cb, float limit, void* ws, size_t ws_bytes, hipStream_t st) {
    EXL3_REQUIRE(tokens >= 1 && topk >= 1, "%s: tokens=%d topk=%d must be >= 1", fn, tokens, topk);
    EXL3_REQUIRE(E >= 1 && E <= kMoeMaxExperts, "%s: num_experts=%d outside 1..%d", fn, E, kMoeMaxExperts);
    EXL3_REQUIRE(topk <= kMoePrefillChunk, "%s: topk=%d above %d", fn, topk, kMoePrefillChunk);
    EXL3_REQUIRE(hidden > 0 && inter > 0 && hidden % 128 == 0 && inter % 128 == 0,
                 "%s: hidden=%d inter=%d must be positive multiples of 128", fn, hidden, inter);
    EXL3_REQUIRE(KG >= 1 && KG <= 8 && KU >= 1 && KU <= 8 && KD >= 1 && KD <= 8,
                 "%s: K (gate %d, up %d, down %d) outside 1..8", fn, KG, KU, KD);
    EXL3_REQUIRE(cb >= 0 && cb <= 2, "%s: codebook=%d outside 0..2", fn, cb);
    bool tabs_ok = true;
    for (int j = 0; j < 9; ++j) tabs_ok = tabs_ok && tb.t[j];
    EXL3_REQUIRE(x && ids && weights && out && tabs_ok, "%s: null pointer", fn);
    EXL3_REQUIRE(aligned(x, 4) && aligned(out, 4), "%s: misaligned x/out", fn);
    if (moe_use_prefill(tokens, topk, E))
        return run_moe_prefill(fn, x, ids, weights, weights_f16, tb, E, out, tokens, topk, hidden, inter, KG, KU, KD,
                               cb, limit, ws, ws_bytes, st);
    return run_moe_decode(fn, x, ids, weights, weights_f16, tb, E, out, tokens, topk, hidden, inter, KG, KU, KD, cb,
                          limit, ws, ws_bytes, st);
}

}  // namespace
}  // namespace exl3

using namespace exl3;

extern "C" size_t exl3_moe_workspace_size(int tokens, int topk, int num_experts, int hidden, int inter) {
    if (tokens < 1 || topk < 1 || num_experts < 1 || hidden < 128 || inter < 128) return 0;
    if (moe_use_prefill(tokens, topk, num_experts)) return prefill_layout(tokens, topk, num_experts, hidden, inter).total;
    return moe_layout(tokens, topk, num_experts, hidden, inter).total;
}

extern "C" int exl3_moe_plan(int tokens, int topk, int num_experts, int hidden, int inter, int* out) {
    clear_error();
    EXL3_REQUIRE(out, "exl3_moe_plan: null pointer");
    EXL3_REQUIRE(tokens >= 1 && topk >= 1 && num_experts >= 1 && hidden >= 128 && inter >= 128 &&
                     hidden % 128 == 0 && inter % 128 == 0,
                 "exl3_moe_plan: bad shape");
    const MoeLayout L = moe_layout(tokens, topk, num_experts, hidden, inter);
    const MoePlan* pls[2] = {&L.gu, &L.dn};
    for (int j = 0; j < 2; ++j) {
        out[4 * j + 0] = pls[j]->bpi;
        out[4 * j + 1] = pls[j]->ns;
        out[4 * j + 2] = pls[j]->kw;
        out[4 * j + 3] = pls[j]->splits;
    }
    out[8] = L.max_units;
    return EXL3_OK;
}

extern "C" int exl3_moe_layer(const uint16_t* x, const int32_t* topk_ids, const float* topk_weights,
                              const int64_t* gate_trellis, const int64_t* gate_suh, const int64_t* gate_svh,
                              const int64_t* up_trellis, const int64_t* up_suh, const int64_t* up_svh,
                              const int64_t* down_trellis, const int64_t* down_suh, const int64_t* down_svh,
                              int num_experts, uint16_t* out, int tokens, int topk, int hidden, int inter,
                              int K_gate, int K_up, int K_down, int codebook, float swiglu_limit,
                              void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    MoeTables tb{{gate_trellis, gate_suh, gate_svh, up_trellis, up_suh, up_svh, down_trellis, down_suh, down_svh}};
    return run_moe("exl3_moe_layer", x, topk_ids, topk_weights, 0, tb, num_experts, out, tokens, topk, hidden,
                   inter, K_gate, K_up, K_down, codebook, swiglu_limit, workspace, workspace_bytes,
                   as_stream(stream));
}

extern "C" int exl3_p2b_fused_moe(const uint16_t* x, uint16_t* out, const int64_t* gate_trellis,
                                  const int64_t* gate_suh, const int64_t* gate_svh, const int64_t* up_trellis,
                                  const int64_t* up_suh, const int64_t* up_svh, const int64_t* down_trellis,
                                  const int64_t* down_suh, const int64_t* down_svh, int num_experts,
                                  const int32_t* expert_ids, const uint16_t* routing_weights, int num_ids,
                                  int hidden, int inter, int K_gate, int K_up, int K_down, int codebook,
                                  float swiglu_limit, void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    MoeTables tb{{gate_trellis, gate_suh, gate_svh, up_trellis, up_suh, up_svh, down_trellis, down_suh, down_svh}};
    return run_moe("exl3_p2b_fused_moe", x, expert_ids, routing_weights, 1, tb, num_experts, out, 1, num_ids,
                   hidden, inter, K_gate, K_up, K_down, codebook, swiglu_limit, workspace, workspace_bytes,
                   as_stream(stream));
}
