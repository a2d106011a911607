// Batched routed-expert MoE layer for gfx950: every active expert of a batch
// of tokens in two to five launches, with no host synchronisation (one token:
// gate/up and down only, routed directly; from 2 tokens the routing kernel,
// which also rotates the gate/up inputs; the separate combine above 48).  Opt-in,
// gate/up and down also run as one persistent launch (moe_fused_direct_kernel
// for one token, moe_fused_routed_kernel after the routing launch).
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
//            adds w * y of each row into its token's fixed-point output
//            accumulators, the add completing a token writing its fp16 row
//            (deterministic: integer sums); without room for the
//            accumulators it stores each row at its (token, slot) entry and
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
// Kernel variants (compile-time, so each holds only its own code path):
constexpr int MV_GU = 0;         // gate/up, input rows rotated by each item
constexpr int MV_GU_ROT = 1;     // gate/up, input rows arrive rotated per projection
constexpr int MV_DOWN = 2;       // down, input rows arrive rotated
constexpr int MV_GU_DIRECT = 3;  // MV_GU for one token routed directly (no routing kernel)
constexpr int MV_DOWN_DIRECT = 4;  // MV_DOWN for one token routed directly
constexpr int MOE_ROUTE_THREADS = 1024;
constexpr int MOE_UNIT_ROWS = 16;  // rows of a work unit: one MFMA row block
constexpr int MV_PRE = 2;          // staged blocks per wave whose activations are loaded up front

// A work unit: up to 16 rows of one expert, with the expert's weight
// addresses resolved by the routing kernel (one dependent load for the GEMV
// workgroups instead of slot -> expert -> table chains).
struct alignas(16) MoeUnit {
    int nrows;            // 1..16
    int crow0;            // first compact row (rows of one expert are contiguous)
    int e;                // expert id
    int pad;
    const void* ptr[9];   // gate trellis/suh/svh, up trellis/suh/svh, down trellis/suh/svh
    long long pad2;
};
static_assert(sizeof(MoeUnit) == 96, "MoeUnit layout");

// Per-expert weight address tables (int64 device arrays indexed by expert id,
// the layout of src/sglang_exl3/exl3.py:590-607).
struct MoeTables {
    const int64_t* t[9];  // gate trellis/suh/svh, up ..., down ...
};

// Device arrays written by moe_route_kernel (inside the caller's workspace).
struct MoeRoute {
    int* counts;     // [0] active experts, [1] work units
    MoeUnit* units;  // [max units]
    int* rows;       // [entries] compact row -> entry index (token * topk + slot)
};

struct MoeParams {
    MoeRoute rt;
    int topk;
    int entries;       // tokens * topk
    int single_token;  // every entry reads x row 0 (one token)
    const __half* x;   // GATE_UP: tokens [T][k]; DOWN: rotated activations [entries][k] by compact row
    float limit;       // SwiGLU clamp; <= 0 or inf: none
    __half* out;       // GATE_UP: [entries][n] by compact row; DOWN: [entries][n] by entry
    float* partials;   // [n/128][nproj][S][entries][128]
    int* counters;     // [units][n/128]
    int k, n;
    int nproj;         // projections summed by the epilogue (2 gate/up, 1 down)
    int proj_base;     // first projection this launch enumerates
    int proj_launch;   // projections this launch enumerates (1 or 2)
    int splits;        // S
    int kw;            // k waves per workgroup
    int bx_per_item;   // column blocks one item covers (divides n/128)
    int bpi_dyn;       // routed launches: the kernel sets bx_per_item from the unit count (moe_item_bpi)
    int mode;
    int in_rot;        // GATE_UP: x holds the rows already rotated per projection,
                       // [2][entries][k] by (token, slot) entry (moe_route_rotate_kernel)
    // DOWN with the weighted combine fused (fc != 0): each row's w[entry] * y
    // is added into 64-bit fixed-point accumulators acc[token][n]; the add that
    // completes the token's valid-slot count writes the fp16 output and clears
    // the accumulator (integer addition: the result does not depend on the
    // order of arrival)
    int fc;
    unsigned long long* acc;  // [tokens][n], zero between calls
    const int* tok_valid;     // [tokens] valid slots per token (routing kernel)
    const void* weights;      // [entries] routing weights, fp16 or fp32
    int weights_f16;
    __half* final_out;        // [tokens][n]
    // One token routed directly, without the routing kernel: unit u is slot u
    // (one row, compact row u, entry u) with its weights looked up in tabs;
    // slots whose id is outside [0, E) are skipped.
    int direct;
    const int32_t* ids;
    int E;
    MoeTables tabs;
    // Gate/up and down in one launch (moe_fused_direct_kernel): readiness
    // flags of the h blocks [units][ready_nblk] and per-unit counts of down
    // items past their wait, both in the workspace's zeroed counter region.
    int* ready;
    int* done;
    int ready_nblk;
    int ready_stride;  // ints between the flag rows of two units
    int poll_sleep;    // s_sleep(8) calls between two polls
    int prime_late;    // down items request their weights after the wait
    int dn_items_per_unit;
    int ready_target;  // count that marks an h block ready: 1, or 2 S (split fixed-point gate/up)
    // Down pass with the fused combine, one round trip per split (fxs != 0,
    // moe_gemv_kernel<.., FXS = true>): each k-split item rotates and scales
    // its own partial rows and adds w * svh * H(partial) / sqrt(128) straight
    // into the token's fixed-point accumulators, which complete after
    // valid-slots x splits contributions (the output rotation is linear).
    int fxs;
    // Bounded waits (fused one-token launch): polls before a wait gives up,
    // and the workspace status word that then gets EXL3_WAIT_MOE_FUSED; the
    // launch's tickets (next item, finished workgroups) in the zeroed
    // counter region.
    int max_polls;
    int* status;
    int* ticket;
    // Directly routed items load their pointer-table entries for every
    // expert beside the routed id (up to kDirectTabExperts experts)
    int tab_prefetch;
    // Gate/up by split fixed-point adds (gfx != 0, moe_gemv_kernel<.., FXS =
    // true, GFX = true>): each k-split item rotates and scales its partial
    // rows and adds svh * H(partial) / sqrt(128) into acc[proj][crow][n]; the
    // add completing an element (S contributions) writes the fp16 gate or up
    // output to out[proj][crow][n] and clears it.  The down pass (GFX = true)
    // then stages fp16(silu(min(g, L)) * clamp(u, -L, L)), rotated with its
    // own suh, from those rows.
    int gfx;
};

inline size_t moe_route_smem_bytes(int E, int entries, int tokens) {
    return (size_t)(3 * E + entries + tokens) * sizeof(int);
}

// ------------------------------------------------------------ expert GEMVs

// Wave-uniform values read from memory by vector loads, moved to scalar
// registers (they would otherwise occupy a VGPR per lane).
__device__ __forceinline__ int uniform_i(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ const void* uniform_p(const void* p) {
    const unsigned long long u = reinterpret_cast<unsigned long long>(p);
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)u), hi = __builtin_amdgcn_readfirstlane((unsigned)(u >> 32));
    return reinterpret_cast<const void*>(((unsigned long long)hi << 32) | lo);
}

__device__ __forceinline__ __half2 ld_h2_ptr(const void* base, int idx) {
    return ld_h2(gptr(reinterpret_cast<const __half*>(base)) + idx);
}

// fp16 pair through a device-coherent 32-bit load / store (data handed from
// one workgroup to another inside a launch).
__device__ __forceinline__ __half2 ld_h2_coherent(const EXL3_GLOBAL __half* ptr) {
    const uint32_t u = __hip_atomic_load(reinterpret_cast<uint32_t*>(const_cast<__half*>((const __half*)ptr)),
                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return *reinterpret_cast<const __half2*>(&u);
}
__device__ __forceinline__ void st_h2_coherent(EXL3_GLOBAL __half* ptr, __half2 v) {
    __hip_atomic_store(reinterpret_cast<uint32_t*>((__half*)ptr), *reinterpret_cast<const uint32_t*>(&v),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// fp16(silu(min(g, L)) * clamp(u, -L, L)) of an fp16 gate and up pair (no
// clamp when L <= 0 or infinite).
__device__ __forceinline__ __half2 swiglu_h2(__half2 g, __half2 u, float limit) {
    float g0 = __low2float(g), g1 = __high2float(g), u0 = __low2float(u), u1 = __high2float(u);
    if (limit > 0.0f && limit < __builtin_huge_valf()) {
        g0 = fminf(g0, limit);
        g1 = fminf(g1, limit);
        u0 = fminf(fmaxf(u0, -limit), limit);
        u1 = fminf(fmaxf(u1, -limit), limit);
    }
    return h2_rn(silu_f(g0) * u0, silu_f(g1) * u1);
}

// Wait until the readiness counts f[j0..j1] all reach `target` (one thread),
// for at most max_polls polls (each followed by nsleep s_sleep(8) calls, ~0.2
// us each): a bound so that every wave exits even if a producer never ran.
// Returns false when the wait gave up.
__device__ __forceinline__ bool wait_ready(const int* f, int j0, int j1, int target, int nsleep, int max_polls) {
    for (int it = 0; it < max_polls; ++it) {
        bool ok = true;
        for (int j = j0; j <= j1; ++j)
            ok = ok && __hip_atomic_load(const_cast<int*>(f) + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= target;
        if (ok) return true;
        for (int z = 0; z < nsleep; ++z) __builtin_amdgcn_s_sleep(8);
    }
    return false;
}

// Experts up to which a directly routed item loads its pointer-table entries
// for every expert alongside the routed id (4 per lane).
constexpr int kDirectTabExperts = 256;

// Entries lane, lane + 64, lane + 128, lane + 192 of a pointer table (0 past E).
struct TabRow {
    unsigned long long v0, v1, v2, v3;
};
__device__ __forceinline__ TabRow tab_row(const int64_t* t, int E, int lane) {
    const EXL3_GLOBAL int64_t* g = gptr(t);
    TabRow r;
    r.v0 = lane < E ? (unsigned long long)g[lane] : 0ull;
    r.v1 = lane + 64 < E ? (unsigned long long)g[lane + 64] : 0ull;
    r.v2 = lane + 128 < E ? (unsigned long long)g[lane + 128] : 0ull;
    r.v3 = lane + 192 < E ? (unsigned long long)g[lane + 192] : 0ull;
    return r;
}
// Entry e (uniform, < 256) of a TabRow, as a wave-uniform pointer.
__device__ __forceinline__ const void* tab_pick(const TabRow& r, int e) {
    const int s = e >> 6;
    const unsigned long long v = s == 0 ? r.v0 : (s == 1 ? r.v1 : (s == 2 ? r.v2 : r.v3));
    const unsigned lo = __builtin_amdgcn_readlane((unsigned)v, e & 63);
    const unsigned hi = __builtin_amdgcn_readlane((unsigned)(v >> 32), e & 63);
    return reinterpret_cast<const void*>(((unsigned long long)hi << 32) | lo);
}

// Valid slots of a directly routed token (ids in [0, E)).
__device__ __forceinline__ int direct_valid_slots(const MoeParams& p) {
    int v = 0;
    for (int sl = 0; sl < p.topk; ++sl) {
        const int e = uniform_i(gptr(p.ids)[sl]);
        v += e >= 0 && e < p.E;
    }
    return v;
}

// fp16 zero row of n columns (workgroup-wide).
__device__ __forceinline__ void zero_row(__half* out, int n) {
    for (int c = threadIdx.x; c < n / 2; c += blockDim.x) reinterpret_cast<EXL3_GLOBAL uint32_t*>(gptr(out))[c] = 0u;
}

// One work item (unit, column block group, projection, k-split) of a
// projection pass: stage the unit's activation rows (rotated by the
// projection's suh unless the input arrives rotated), decode + MFMA the
// split's k range for each of the group's 128-column blocks, store fp32
// partial rows; the last of nproj * S arrivals of (unit, column block) runs
// the epilogue.  `first`: this is the workgroup's first item (no barrier for
// the LDS of a previous one).  FUSED: the gate/up and down passes share one
// launch (moe_fused_direct_kernel): gate/up epilogues publish each finished
// 128-wide block of h, and down items wait for the blocks they read.
template <int K, int CB, int NS, int MODE, int KW, bool FUSED, bool FXS = false, bool GFX = false>
__device__ __forceinline__ void moe_item(const MoeParams& p, int it, unsigned char* mv_smem, int direct_valid,
                                         bool first, int bpi) {
    constexpr int ROWS = MOE_UNIT_ROWS;
    __shared__ int is_last;
    constexpr bool direct = MODE == MV_GU_DIRECT || MODE == MV_DOWN_DIRECT;
    const int nblk_n = p.n >> 7;
    const int BPI = bpi, ngroups = nblk_n / BPI;
    const int S = p.splits, P = p.proj_launch;
    const int per_unit = ngroups * P * S;
    const int k = p.k, n = p.n;
    constexpr int kw = KW;  // k waves (p.kw)
    constexpr int nsteps = NS;
    const int nthreads = 256 * kw, nwaves = 4 * kw;
    const int kts_wg = 4 * nsteps * kw;
    const int ntiles = n >> 4;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int cw = wave & 3, kwi = wave >> 2;
    const int g = lane >> 4, i = lane & 15, q = i & 7;
    constexpr bool down = MODE == MV_DOWN || MODE == MV_DOWN_DIRECT;
    // input rows arrive rotated (a GFX down pass rotates the SwiGLU it stages)
    constexpr bool pre_rotated = MODE != MV_GU && MODE != MV_GU_DIRECT && !(down && GFX);
    static_assert(!GFX || FXS, "split fixed-point gate/up: FXS items");
    const size_t step_stride = (size_t)4 * ntiles * (8 * K);
    const size_t split_stride = (size_t)p.entries * 128;
    const int nblk128 = kts_wg >> 3;
    _Float16* xs = reinterpret_cast<_Float16*>(mv_smem);
    const int xs_halves = kts_wg * 4 * ROWS * 8;
    float* xsum = reinterpret_cast<float*>(mv_smem + (((size_t)xs_halves * 2 + 16 + 15) & ~(size_t)15));
    float* ybuf = xsum + ((ROWS * nblk128 + 3) & ~3);
    if (tid < 8) xs[xs_halves + tid] = (_Float16)0.0f;
    const EXL3_GLOBAL int* rows_g = gptr(p.rt.rows);

    const int u = it / per_unit;
    int rem = it - u * per_unit;
    const int bg = rem / (P * S);
    rem -= bg * P * S;
    const int pl = rem / S, sidx = rem - pl * S;
    const int proj = p.proj_base + pl;

    const int pb = down ? 6 : 3 * proj;
    int m, crow0;
    const void *tp, *suh, *ev0p, *ev1p, *ev2p;
    if (direct) {
        // Up to kDirectTabExperts experts, the table entries this item reads
        // are requested for every expert (entry lane + 64 s in lane `lane`)
        // together with the routed id, so the weight and sign-vector loads
        // wait for one round trip instead of two (id, then entry).
        const bool pre = p.tab_prefetch && p.E <= kDirectTabExperts;
        const TabRow r0 = pre ? tab_row(p.tabs.t[pb], p.E, lane) : TabRow{};
        const TabRow r1 = pre ? tab_row(p.tabs.t[pb + 1], p.E, lane) : TabRow{};
        const TabRow r2 = pre ? tab_row(p.tabs.t[down ? 8 : 2], p.E, lane) : TabRow{};
        const TabRow r3 = (pre && !down) ? tab_row(p.tabs.t[5], p.E, lane) : TabRow{};
        const TabRow r4 = (pre && !down) ? tab_row(p.tabs.t[7], p.E, lane) : TabRow{};
        const int e = uniform_i(gptr(p.ids)[u]);
        if (e < 0 || e >= p.E) return;  // skipped slot (uniform over the workgroup)
        m = 1;
        crow0 = u;
        auto tab = [&](const TabRow& r, int j) -> const void* {
            return pre ? tab_pick(r, e) : uniform_p(reinterpret_cast<const void*>(gptr(p.tabs.t[j])[e]));
        };
        tp = tab(r0, pb);
        suh = tab(r1, pb + 1);
        ev0p = tab(r2, down ? 8 : 2);
        ev1p = down ? nullptr : tab(r3, 5);
        ev2p = down ? nullptr : tab(r4, 7);
    } else {
        const EXL3_GLOBAL MoeUnit* ud = gptr(p.rt.units) + u;
        m = uniform_i(ud->nrows);
        crow0 = uniform_i(ud->crow0);
        tp = uniform_p(ud->ptr[pb]);
        suh = uniform_p(ud->ptr[pb + 1]);
        ev0p = uniform_p(ud->ptr[down ? 8 : 2]);  // svh of down / gate
        ev1p = uniform_p(ud->ptr[5]);             // svh of up
        ev2p = uniform_p(ud->ptr[7]);             // suh of down (its input rotation)
    }
    const uint32_t* trellis = reinterpret_cast<const uint32_t*>(tp);
    const int kt_wg0 = sidx * kts_wg;
    const int kt_w0 = kt_wg0 + kwi * 4 * nsteps;
    const int bx0 = bg * BPI;
    auto tiles = [&](int bx) {
        return gptr(trellis) + ((size_t)(kt_w0 + g) * ntiles + bx * 8 + cw * 2 + (i >> 3)) * (8 * K) + K * q;
    };
    if (!first) __syncthreads();  // the previous item is done with LDS

    // the entries of the unit's rows, one per lane, looked up once (the
    // row loops below read them with readlane instead of a dependent load
    // per row)
    const bool by_entry = !down && !direct && (pre_rotated || !p.single_token);
    const int ent_lane = (by_entry && lane < m) ? rows_g[crow0 + lane] : 0;
    auto x_row = [&](int row) -> const EXL3_GLOBAL __half* {
        if (down) return gptr(p.x) + (size_t)(crow0 + row) * k;
        if (!by_entry) return gptr(p.x);
        const int entry = __builtin_amdgcn_readlane(ent_lane, row);
        if (pre_rotated) return gptr(p.x) + ((size_t)proj * p.entries + entry) * k;
        return gptr(p.x) + (size_t)(entry / p.topk) * k;
    };

    // 1. activation loads (up to MV_PRE blocks per wave, all in flight),
    //    then the first column block's weights.  A down item of the fused
    //    launch requests its weights first, then waits until the gate/up
    //    epilogues have published the h blocks of its k range (their
    //    stores were device-coherent, so it reads them coherently too).
    constexpr bool wait_h = FUSED && down;
    auto ld_x = [&](const EXL3_GLOBAL __half* ptr) -> __half2 {
        if constexpr (wait_h) return ld_h2_coherent(ptr);
        else return ld_h2(ptr);
    };
    const int nrot = m * nblk128;
    // GFX down pass: x holds the fp16 gate rows, the up rows follow them
    const size_t up_rows = (down && GFX) ? (size_t)p.entries * k : 0;
    __half2 xpre[MV_PRE], spre[MV_PRE], upre[MV_PRE];
    auto preload = [&]() {
#pragma unroll
        for (int j = 0; j < MV_PRE; ++j) {
            const int b = wave + j * nwaves;
            if (b < nrot) {
                const int row = b / nblk128, bb = b - row * nblk128;
                const int kg = kt_wg0 * 16 + bb * 128 + 2 * lane;
                xpre[j] = ld_x(x_row(row) + kg);
                if constexpr (down && GFX) upre[j] = ld_x(x_row(row) + up_rows + kg);
                if (!pre_rotated) spre[j] = ld_h2_ptr(suh, kg);
            }
        }
    };
    // Rows that arrive rotated (read plainly, not by the fused launch's
    // coherent loads): each lane loads its V = NS * KW consecutive k values of
    // a row (kts_wg * 16 / 64) with one set of loads, all of the wave's rows
    // at once, so staging costs one round trip (the block-at-a-time loop
    // below waits a round trip per (row, 128-block) after the first two:
    // up to ~9 us for a 16-row unit at B = 16).  Chunks of 128 % V != 0 with
    // mul1 chunk sums stay on that loop.
    constexpr int V = NS * KW;
    constexpr int RPW = (MOE_UNIT_ROWS + 4 * KW - 1) / (4 * KW);  // rows per wave at most
    constexpr bool vec_stage = pre_rotated && !wait_h && V % 2 == 0 && V <= 16 && (CB != 2 || 128 % V == 0);
    uint32_t xw[vec_stage ? RPW : 1][vec_stage ? V / 2 : 1];
    auto vec_load = [&]() {
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const int row = wave + r * nwaves;
            if (row < m) {
                const EXL3_GLOBAL uint32_t* src =
                    reinterpret_cast<const EXL3_GLOBAL uint32_t*>(x_row(row) + kt_wg0 * 16 + lane * V);
                if constexpr (V % 8 == 0) {
#pragma unroll
                    for (int c = 0; c < V / 8; ++c) {
                        const u32x4_t q = reinterpret_cast<const EXL3_GLOBAL u32x4_t*>(src)[c];
                        xw[r][4 * c] = q.x;
                        xw[r][4 * c + 1] = q.y;
                        xw[r][4 * c + 2] = q.z;
                        xw[r][4 * c + 3] = q.w;
                    }
                } else {
#pragma unroll
                    for (int c = 0; c < V / 2; ++c) xw[r][c] = src[c];
                }
            }
        }
    };
    uint32_t w[gv_depth<K>()][K];
    if constexpr (vec_stage) {
        vec_load();
        prime_weights<K, NS>(w, tiles(bx0), step_stride);
    } else if constexpr (wait_h) {
        if (!p.prime_late) prime_weights<K, NS>(w, tiles(bx0), step_stride);
        if (tid == 0 && !wait_ready(p.ready + (size_t)u * p.ready_stride, kt_wg0 >> 3, (kt_wg0 + kts_wg - 1) >> 3,
                                    p.ready_target, p.poll_sleep, p.max_polls))
            report_wait_expired(p.status, EXL3_WAIT_MOE_FUSED);
        __syncthreads();
        if (p.prime_late) prime_weights<K, NS>(w, tiles(bx0), step_stride);
        preload();
    } else {
        preload();
        prime_weights<K, NS>(w, tiles(bx0), step_stride);
    }

    // 2. stage the rows in A-fragment order once for all column blocks of
    //    the item (rotated here unless they arrive rotated)
    // values kk and kk + 1 of a lane sit at xs_index(kk) and xs_index(kk) + 2
    // (8-byte aligned), so (a, a, c, c) is one 64-bit LDS store
    auto stage = [&](int b, __half2 xv, __half2 uv, __half2 sv) {
        const int row = b / nblk128, bb = b - row * nblk128;
        const int kk = bb * 128 + 2 * lane;
        if constexpr (down && GFX) xv = swiglu_h2(xv, uv, p.limit);
        uint32_t bits;
        if (pre_rotated) {
            bits = *reinterpret_cast<const uint32_t*>(&xv);
        } else {
            const __half2 pr = __hmul2(xv, sv);
            float fa = __low2float(pr), fc = __high2float(pr);
            fwht128_pair_fast(fa, fc, lane);
            const _Float16 ha = f16_rn(fa * kHadNorm), hc = f16_rn(fc * kHadNorm);
            bits = (uint32_t)__builtin_bit_cast(unsigned short, ha) |
                   ((uint32_t)__builtin_bit_cast(unsigned short, hc) << 16);
        }
        const uint32_t da = __builtin_amdgcn_perm(bits, bits, 0x01000100u);  // (a, a)
        const uint32_t dc = __builtin_amdgcn_perm(bits, bits, 0x03020302u);  // (c, c)
        *reinterpret_cast<uint2*>(xs + xs_index(kk, row, kts_wg)) = make_uint2(da, dc);
        if constexpr (CB == 2) {
            const float t = wave_sum(__half2float(__ushort_as_half((unsigned short)(bits & 0xffffu))) +
                                     __half2float(__ushort_as_half((unsigned short)(bits >> 16))));
            if (lane == 0) xsum[b] = t;
        }
    };
    if constexpr (vec_stage) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const int row = wave + r * nwaves;
            if (row < m) {
                float sx = 0.f;
#pragma unroll
                for (int c = 0; c < V / 2; ++c) {
                    const uint32_t bits = xw[r][c];
                    const uint32_t da = __builtin_amdgcn_perm(bits, bits, 0x01000100u);  // (a, a)
                    const uint32_t dc = __builtin_amdgcn_perm(bits, bits, 0x03020302u);  // (c, c)
                    *reinterpret_cast<uint2*>(xs + xs_index(lane * V + 2 * c, row, kts_wg)) = make_uint2(da, dc);
                    if constexpr (CB == 2)
                        sx += __half2float(__ushort_as_half((unsigned short)(bits & 0xffffu))) +
                              __half2float(__ushort_as_half((unsigned short)(bits >> 16)));
                }
                if constexpr (CB == 2) {
                    // chunk sum over the 128 / V lanes of each 128-wide block
#pragma unroll
                    for (int o = 1; o < 128 / V; o <<= 1) sx += __shfl_xor(sx, o);
                    if ((lane & (128 / V - 1)) == 0) xsum[row * nblk128 + lane * V / 128] = sx;
                }
            }
        }
    } else {
#pragma unroll
    for (int j = 0; j < MV_PRE; ++j) {
        const int b = wave + j * nwaves;
        if (b < nrot) stage(b, xpre[j], (down && GFX) ? upre[j] : __half2{}, spre[j]);
    }
    for (int b = wave + MV_PRE * nwaves; b < nrot; b += nwaves) {
        const int row = b / nblk128, bb = b - row * nblk128;
        const int kg = kt_wg0 * 16 + bb * 128 + 2 * lane;
        const __half2 sv = pre_rotated ? __half2{} : ld_h2_ptr(suh, kg);
        const __half2 uv = (down && GFX) ? ld_x(x_row(row) + up_rows + kg) : __half2{};
        stage(b, ld_x(x_row(row) + kg), uv, sv);
    }
    }
    __syncthreads();
    if constexpr (wait_h && FXS) {
        // a fused down item with split fixed-point adds has read its h rows:
        // count it done; the unit's last down item clears the unit's
        // readiness counts for the next call
        if (tid == 0 && __hip_atomic_fetch_add(p.done + u, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                            p.dn_items_per_unit - 1) {
            for (int j = 0; j < p.ready_nblk; ++j)
                __hip_atomic_store(p.ready + (size_t)u * p.ready_stride + j, 0, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(p.done + u, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }

    const bool live = i < m;
    const _Float16* a_base[1] = {xs + (size_t)((live ? i : 0) * kts_wg + kwi * 4 * nsteps + g) * 4 * 8};
    const bool a_live[1] = {live};
    for (int bx = bx0; bx < bx0 + BPI; ++bx) {
        if (bx != bx0) {
            __syncthreads();  // the previous block is done with ybuf
            prime_weights<K, NS>(w, tiles(bx), step_stride);
        }
        // epilogue vectors of this block, requested now so they are in
        // registers at the end
        const int c0 = bx * 128 + 2 * lane;
        // (GFX gate/up: only the item's own projection's svh)
        const __half2 ev0 = ld_h2_ptr((GFX && !down && proj == 1) ? ev1p : ev0p, c0);
        __half2 ev1 = __half2{}, ev2 = __half2{};
        if (!down && !GFX) {
            ev1 = ld_h2_ptr(ev1p, c0);
            ev2 = ld_h2_ptr(ev2p, c0);
        }

        // 3. decode + MFMA (rows >= m read nothing and multiply zeros)
        float4_t acc[1][2];
        acc[0][0] = float4_t{0.f, 0.f, 0.f, 0.f};
        acc[0][1] = float4_t{0.f, 0.f, 0.f, 0.f};
        decode_mfma_steps<K, CB, 1, NS>(w, tiles(bx), step_stride, a_base, a_live, acc);

        if constexpr (FXS) {
            static_assert(KW == 1 && (down || GFX), "split fixed-point adds: down pass, or gate/up with GFX");
            // the four waves' column slices of the unit's rows meet in LDS
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = 4 * g + r;
                if (row >= m) continue;
#pragma unroll
                for (int c = 0; c < 2; ++c) ybuf[row * 128 + cw * 32 + (i >> 3) * 16 + (i & 7) + 8 * c] = acc[0][c][r];
            }
            __syncthreads();
            // one row per wave: mul1 map, output rotation, svh, routing
            // weight, then the adds; a row's adds are checked after the next
            // row's have been issued, so their round trips overlap
            FxPair fx{};
            int ptok = -1, pcnt = 0;
            size_t pofs = 0;  // gate/up: the pending pair's element offset
            for (int row = wave; row < m; row += nwaves) {
                float va = ybuf[row * 128 + 2 * lane], vb = ybuf[row * 128 + 2 * lane + 1];
                if constexpr (CB == 2) {
                    float sx = 0.f;
                    for (int bb = 0; bb < nblk128; ++bb) sx += xsum[row * nblk128 + bb];
                    va = va * kMul1Kinv + kMul1Delta * sx;
                    vb = vb * kMul1Kinv + kMul1Delta * sx;
                }
                fwht128_pair_fast(va, vb, lane);
                const int crow = crow0 + row;
                if constexpr (!down) {
                    // gate or up element (proj, crow, col): S contributions
                    const size_t o = ((size_t)proj * p.entries + crow) * n + c0;
                    const FxPair cur =
                        fx_issue_pair(p.acc + o, (va * kHadNorm) * __low2float(ev0), (vb * kHadNorm) * __high2float(ev0));
                    if (ptok >= 0) fx_finish_pair<FUSED>(fx, p.acc + pofs, S, gptr(p.out) + pofs);
                    fx = cur;
                    pofs = o;
                    ptok = 0;
                    continue;
                }
                const int entry = direct ? crow : uniform_i(rows_g[crow]);
                const int t = entry / p.topk;
                const float wv = p.weights_f16
                                     ? __half2float(__ushort_as_half(gptr(reinterpret_cast<const uint16_t*>(p.weights))[entry]))
                                     : gptr(reinterpret_cast<const float*>(p.weights))[entry];
                const int c = (direct ? direct_valid : uniform_i(gptr(p.tok_valid)[t])) * S;
                const float sa = wv * kHadNorm * __low2float(ev0), sb = wv * kHadNorm * __high2float(ev0);
                const FxPair cur = fx_issue_pair(p.acc + (size_t)t * n + c0, va * sa, vb * sb);
                if (ptok >= 0)
                    fx_finish_pair(fx, p.acc + (size_t)ptok * n + c0, pcnt, gptr(p.final_out) + (size_t)ptok * n + c0);
                fx = cur;
                ptok = t;
                pcnt = c;
            }
            if constexpr (!down) {
                if (ptok >= 0) fx_finish_pair<FUSED>(fx, p.acc + pofs, S, gptr(p.out) + pofs);
                if constexpr (FUSED) {
                    // this item's share of the block's gate or up elements is
                    // in (and the elements it completed are stored): count it
                    // toward the block's 2 S
                    wait_stores();
                    __syncthreads();
                    if (tid == 0)
                        __hip_atomic_fetch_add(p.ready + (size_t)u * p.ready_stride + bx, 1, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
                }
            } else if (ptok >= 0) {
                fx_finish_pair(fx, p.acc + (size_t)ptok * n + c0, pcnt, gptr(p.final_out) + (size_t)ptok * n + c0);
            }
            continue;
        }

        // 4. k waves summed through LDS, mul1 affine map, partial rows out
        //    (one k wave: straight from the accumulators, no LDS tile, so
        //    four workgroups fit a CU)
        float* part =
            p.partials + ((size_t)(bx * p.nproj + proj) * S + sidx) * split_stride + (size_t)crow0 * 128;
        if constexpr (KW == 1) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = 4 * g + r;
                if (row >= m) continue;
                float sx = 0.f;
                if constexpr (CB == 2)
                    for (int bb = 0; bb < nblk128; ++bb) sx += xsum[row * nblk128 + bb];
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    const int col = cw * 32 + (i >> 3) * 16 + (i & 7) + 8 * c;
                    float v = acc[0][c][r];
                    if constexpr (CB == 2) v = v * kMul1Kinv + kMul1Delta * sx;
                    coherent_store(part + row * 128 + col, v);
                }
            }
        }
        else {
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = 4 * g + r;
                    const int col = cw * 32 + (i >> 3) * 16 + (i & 7) + 8 * c;
                    if (row < m) ybuf[(kwi * ROWS + row) * 128 + col] = acc[0][c][r];
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
                coherent_store(part + idx, v);
            }
        }

        // 5. hand-off: the last of nproj * S arrivals for (unit, column
        //    block) finishes
        wait_stores();
        __syncthreads();
        int* ctr = p.counters + (size_t)u * nblk_n + bx;
        if (tid == 0) {
            // a fused down item has read its h rows (staged above): its first
            // hand-off also counts it done, in the same round trip, and the
            // unit's last down item clears the unit's readiness flags for the
            // next call
            int dold = 0;
            if constexpr (wait_h)
                if (bx == bx0) dold = __hip_atomic_fetch_add(p.done + u, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const int old = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            is_last = (old == p.nproj * S - 1);
            if constexpr (wait_h)
                if (bx == bx0 && dold == p.dn_items_per_unit - 1) {
                    for (int j = 0; j < p.ready_nblk; ++j)
                        __hip_atomic_store(p.ready + (size_t)u * p.ready_stride + j, 0, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(p.done + u, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
        }
        __syncthreads();
        if (!is_last) continue;
        if (tid == 0) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

        // 6. epilogue, one row per wave, 2 columns per lane; split partials
        //    of a row are requested in groups of 4 splits before their adds
        //    (one round trip per group) and summed in split order.  Groups of
        //    8 held the gate/up variants at the 128-VGPR cap with spills
        //    (102 VGPRs and none with 4).
        auto sum_rows = [&](int np, int crow, float2* out) {
            constexpr int G = 4;
            for (int s0 = 0; s0 < S; s0 += G) {
                float2 v[2][G];
#pragma unroll
                for (int pj = 0; pj < 2; ++pj)
#pragma unroll
                    for (int j = 0; j < G; ++j)
                        if (pj < np && s0 + j < S)
                            v[pj][j] = coherent_load2(
                                p.partials + ((size_t)(bx * p.nproj + pj) * S + s0 + j) * split_stride +
                                (size_t)crow * 128 + 2 * lane);
#pragma unroll
                for (int pj = 0; pj < 2; ++pj)
#pragma unroll
                    for (int j = 0; j < G; ++j)
                        if (pj < np && s0 + j < S) {
                            out[pj].x += v[pj][j].x;
                            out[pj].y += v[pj][j].y;
                        }
            }
        };
        EXL3_GLOBAL __half* outg = gptr(p.out);
        if (!down) {
            for (int row = wave; row < m; row += nwaves) {
                const int crow = crow0 + row;
                float2 gu[2] = {make_float2(0.f, 0.f), make_float2(0.f, 0.f)};
                sum_rows(2, crow, gu);
                float ga = gu[0].x, gb = gu[0].y, ua = gu[1].x, ub = gu[1].y;
                fwht128_pair_fast(ga, gb, lane);
                fwht128_pair_fast(ua, ub, lane);
                // gate and up outputs in fp16, as the separate linears return them
                const __half2 gh =
                    h2_rn(ga * kHadNorm * __low2float(ev0), gb * kHadNorm * __high2float(ev0));
                const __half2 uh =
                    h2_rn(ua * kHadNorm * __low2float(ev1), ub * kHadNorm * __high2float(ev1));
                const __half2 act = swiglu_h2(gh, uh, p.limit);
                // input rotation of the down projection for this 128-wide chunk
                const __half2 pr = __hmul2(act, ev2);
                float da = __low2float(pr), db = __high2float(pr);
                fwht128_pair_fast(da, db, lane);
                if constexpr (FUSED) st_h2_coherent(outg + (size_t)crow * n + c0, h2_rn(da * kHadNorm, db * kHadNorm));
                else st_h2(outg + (size_t)crow * n + c0, h2_rn(da * kHadNorm, db * kHadNorm));
            }
            if constexpr (FUSED) {
                // the rows of this 128-wide block of h are complete: publish
                // the block to the down items of the same launch
                wait_stores();
                __syncthreads();
                if (tid == 0)
                    __hip_atomic_store(p.ready + (size_t)u * p.ready_stride + bx, 1, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            }
        } else {
            // fused combine: a row's fixed-point adds are checked only
            // after the next row's partials have been loaded, so their
            // round trips overlap
            FxPair fx{};
            int ptok = -1, pcnt = 0;
            for (int row = wave; row < m; row += nwaves) {
                const int crow = crow0 + row;
                float2 d[2] = {make_float2(0.f, 0.f), make_float2(0.f, 0.f)};
                sum_rows(1, crow, d);
                float va = d[0].x, vb = d[0].y;
                fwht128_pair_fast(va, vb, lane);
                const int entry = direct ? crow : uniform_i(rows_g[crow]);
                // the expert's output row in fp16, as the separate linear returns it
                const __half2 yh = h2_rn(va * kHadNorm * __low2float(ev0), vb * kHadNorm * __high2float(ev0));
                if (p.fc) {
                    const int t = entry / p.topk;
                    const float wv =
                        p.weights_f16
                            ? __half2float(__ushort_as_half(
                                  gptr(reinterpret_cast<const uint16_t*>(p.weights))[entry]))
                            : gptr(reinterpret_cast<const float*>(p.weights))[entry];
                    const int c = direct ? direct_valid : uniform_i(gptr(p.tok_valid)[t]);
                    const FxPair cur =
                        fx_issue_pair(p.acc + (size_t)t * n + c0, wv * __low2float(yh), wv * __high2float(yh));
                    if (ptok >= 0)
                        fx_finish_pair(fx, p.acc + (size_t)ptok * n + c0, pcnt,
                                       gptr(p.final_out) + (size_t)ptok * n + c0);
                    fx = cur;
                    ptok = t;
                    pcnt = c;
                } else {
                    st_h2(outg + (size_t)entry * n + c0, yh);
                }
            }
            if (ptok >= 0)
                fx_finish_pair(fx, p.acc + (size_t)ptok * n + c0, pcnt, gptr(p.final_out) + (size_t)ptok * n + c0);
        }
    }
}

// Column blocks per item of a routed pass, from the routed unit count: the
// divisor d <= 4 of the pass's column blocks whose item count lands nearest
// 2.2 rounds of the grid (ties: the smaller d).  The planner sizes items from the
// unit count of uniform routing; a skewed router activates far fewer experts
// (config 4, Zipf 1.1, B = 32: 45 units against 113), and the best grouping
// follows the actual count.  Graph-timed, rounds of the grid -> us: config 4
// Zipf B = 32: 2.1 / 1.06 -> 54.5 / 58.5 (d = 1 / 2); B = 56: 3.0 / 1.5 -> 81.5 /
// 77.7; B = 64: 3.3 / 1.66 / 1.1 -> 89.1 / 81.6 / 88.5 (d = 1 / 2 / 3);
// uniform B = 8: 2.5 / 1.2 -> 51.3 / 57.6; B = 16: 3.8 / 1.9 -> 74.3 / 72.7;
// config 5 gate/up (K = 2): 6.2 / 3.1 / 2.1 / 1.5 -> 102.9 / 104.2 / 100.3 /
// 106.9 (d = 1 / 2 / 3 / 4).  Outputs do not depend on it: each block's
// product is the same.
__device__ __forceinline__ int moe_item_bpi(const MoeParams& p, int nunits, int grid) {
    if (!p.bpi_dyn) return p.bx_per_item;
    const int nblk = p.n >> 7;
    const int per_block = nunits * p.proj_launch * p.splits;
    const int target = 11 * grid;  // 5 x items against 11 x grid: 2.2 rounds
    // candidates d = 1..4 (the divisors that occur at these shapes), the
    // divisions by constants
    int best = 1, best_dev = abs(5 * per_block * nblk - target);
    if (nblk % 2 == 0) {
        const int dev = abs(5 * per_block * (nblk / 2) - target);
        if (dev < best_dev) best = 2, best_dev = dev;
    }
    if (nblk % 3 == 0) {
        const int dev = abs(5 * per_block * (nblk / 3) - target);
        if (dev < best_dev) best = 3, best_dev = dev;
    }
    if (nblk % 4 == 0) {
        const int dev = abs(5 * per_block * (nblk / 4) - target);
        if (dev < best_dev) best = 4, best_dev = dev;
    }
    return best;
}

// Persistent over the work items of one projection pass: the grid is sized
// to the device, the item count comes from the routing kernel (or the slots
// of a directly routed token), so no workgroup is launched for an inactive
// expert.  Items are taken in rounds over the grid, snake order (round r:
// workgroup b takes item r G + b for even r, r G + G - 1 - b for odd r), so
// the workgroup with the last (lightest) item of a round takes the first
// (heaviest) of the next.
template <int K, int CB, int NS, int MODE, int KW, bool FXS = false, bool GFX = false>
__global__ __launch_bounds__(GV_MAX_THREADS, 4) void moe_gemv_kernel(MoeParams p) {
    extern __shared__ __align__(16) unsigned char mv_smem[];
    constexpr bool direct = MODE == MV_GU_DIRECT || MODE == MV_DOWN_DIRECT;
    constexpr bool down = MODE == MV_DOWN || MODE == MV_DOWN_DIRECT;
    const int nunits = direct ? p.topk : uniform_i(gptr(p.rt.counts)[1]);
    // wave-uniform, in a scalar register (the item decomposition divides by it)
    const int bpi = direct ? p.bx_per_item : uniform_i(moe_item_bpi(p, nunits, (int)gridDim.x));
    const int per_unit = ((p.n >> 7) / bpi) * p.proj_launch * p.splits;
    const int total = nunits * per_unit;
    if ((int)blockIdx.x >= total) return;
    // one token routed directly: its valid slots (the fused combine's count);
    // with none, workgroup 0 writes the zero output row
    int direct_valid = 0;
    if (down && direct) {
        direct_valid = direct_valid_slots(p);
        if (direct_valid == 0) {
            if (blockIdx.x == 0 && p.fc) zero_row(p.final_out, p.n);
            return;
        }
    }
    const int G = gridDim.x, b0 = blockIdx.x;
    for (int rnd = 0, it = b0; it < total; ++rnd, it = rnd * G + ((rnd & 1) ? G - 1 - b0 : b0))
        moe_item<K, CB, NS, MODE, KW, false, FXS, GFX>(p, it, mv_smem, direct_valid, rnd == 0, bpi);
}

// One token routed directly, gate/up and down in one persistent launch.
// Items [0, Ngu) are the gate/up items, [Ngu, Ngu + Ndn) the down items.
// Workgroup b takes item b first; when the grid is smaller than the item
// count, further items come from a ticket counter (pg.ticket[0], zero
// between calls) starting at the grid size, so items are taken in index
// order and the last workgroup to finish (pg.ticket[1] counts them) resets
// both counters.  A down item requests its weights at once and then waits
// (bounded) for the h blocks of its k range, which gate/up items (never
// waiting) publish.  Forward progress: a claimed item's gate/up producers
// were claimed earlier; a first-round item's producers are the first items
// of lower-numbered workgroups, which the grid (sized to the workgroups the
// device holds at once) has running beside it.  If other work keeps some of
// them from being resident, the wait gives up and sets EXL3_WAIT_MOE_FUSED in
// the workspace status word.  (Claiming every item from the ticket measured
// 38.4 against 22 us on config 4 B = 1: 768 contended atomics on one word.)
template <int K, int CB, int NSG, int NSD, bool GFX = false>
__global__ __launch_bounds__(GV_MAX_THREADS, 4) void moe_fused_direct_kernel(MoeParams pg, MoeParams pd) {
    extern __shared__ __align__(16) unsigned char mv_smem[];
    __shared__ int claimed;
    const int direct_valid = direct_valid_slots(pd);
    if (direct_valid == 0) {
        if (blockIdx.x == 0 && pd.fc) zero_row(pd.final_out, pd.n);
        return;
    }
    const int ngu = pg.topk * ((pg.n >> 7) / pg.bx_per_item) * pg.proj_launch * pg.splits;
    const int total = ngu + pd.topk * ((pd.n >> 7) / pd.bx_per_item) * pd.splits;
    const int G = gridDim.x;
    for (int rnd = 0, it = blockIdx.x; it < total; ++rnd) {
        if (it < ngu) moe_item<K, CB, NSG, MV_GU_DIRECT, 1, true, GFX, GFX>(pg, it, mv_smem, direct_valid, rnd == 0,
                                                                   pg.bx_per_item);
        else moe_item<K, CB, NSD, MV_DOWN_DIRECT, 1, true, GFX, GFX>(pd, it - ngu, mv_smem, direct_valid, rnd == 0,
                                                                     pd.bx_per_item);
        if (G >= total) break;
        __syncthreads();
        if (threadIdx.x == 0)
            claimed = G + __hip_atomic_fetch_add(pg.ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        it = claimed;
    }
    if (G < total && threadIdx.x == 0 &&
        __hip_atomic_fetch_add(pg.ticket + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == G - 1) {
        __hip_atomic_store(pg.ticket, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(pg.ticket + 1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Routed batch, gate/up and down in one persistent launch over the active
// units (after the routing launch, which also rotates the gate/up inputs).
// Items [0, Ngu) are the gate/up items, [Ngu, Ngu + Ndn) the down items, taken
// in the snake rounds of moe_gemv_kernel.  A gate/up item publishes its h
// blocks (readiness counts per unit and 128-wide block, as in the one-token
// launch); a down item requests its weights, then waits (bounded) for the
// blocks of its k range.  Forward progress: every workgroup is resident (the
// grid is the device's resident capacity), gate/up items never wait, and a
// down item waits only for items of lower index, i.e. of its own round or an
// earlier one, which the other resident workgroups reach without waiting on
// anything later.  If other work keeps workgroups off the device, a wait
// gives up and sets EXL3_WAIT_MOE_FUSED in the workspace status word.  DFX:
// the down pass adds into the fused combine's fixed-point accumulators (one
// round trip per split).  Opt-in: slower than the separate launches.
template <int K, int CB, int NSG, int NSD, bool GFX, bool DFX>
__global__ __launch_bounds__(GV_MAX_THREADS, 4) void moe_fused_routed_kernel(MoeParams pg, MoeParams pd) {
    extern __shared__ __align__(16) unsigned char mv_smem[];
    static_assert(!GFX || DFX, "split fixed-point gate/up: the down pass stages the SwiGLU, FXS items");
    const int nunits = uniform_i(gptr(pg.rt.counts)[1]);
    const int ngu = nunits * ((pg.n >> 7) / pg.bx_per_item) * pg.proj_launch * pg.splits;
    const int total = ngu + nunits * ((pd.n >> 7) / pd.bx_per_item) * pd.splits;
    const int G = gridDim.x, b0 = blockIdx.x;
    for (int rnd = 0, it = b0; it < total; ++rnd, it = rnd * G + ((rnd & 1) ? G - 1 - b0 : b0)) {
        if (it < ngu) moe_item<K, CB, NSG, MV_GU_ROT, 1, true, GFX, GFX>(pg, it, mv_smem, 0, rnd == 0, pg.bx_per_item);
        else moe_item<K, CB, NSD, MV_DOWN, 1, true, DFX, GFX>(pd, it - ngu, mv_smem, 0, rnd == 0, pd.bx_per_item);
    }
}

// Dynamic LDS bytes of moe_gemv_kernel.
// fxs: the split fixed-point down pass, whose one k-wave still meets in an
// LDS tile of the unit's rows.
inline size_t moe_smem_bytes(int kts_wg, int kw, bool fxs = false) {
    const int rows = MOE_UNIT_ROWS;
    const size_t xs = ((size_t)kts_wg * 4 * rows * 8 * 2 + 16 + 15) & ~(size_t)15;
    const size_t tile = kw > 1 ? (size_t)kw * rows * 128 * 4 : (fxs ? (size_t)rows * 128 * 4 : 0);
    return xs + (size_t)((rows * (kts_wg / 8) + 3) & ~3) * 4 + tile;
}

// Workgroups of moe_gemv_kernel<...> the device holds at once (cached).
int moe_grid_size(const void* fn, int threads, size_t smem);

template <int K>
int moe_launch_k(int cb, int ns, const MoeParams& p, hipStream_t st) {
    const bool gfx = p.gfx != 0;
    const bool fxs = p.fxs && p.kw == 1 && (p.mode == MOE_DOWN || gfx);
    const size_t smem = moe_smem_bytes(4 * ns * p.kw, p.kw, fxs);
    const int threads = 256 * p.kw;
    const int mv = p.mode == MOE_DOWN ? (p.direct ? MV_DOWN_DIRECT : MV_DOWN)
                                      : (p.in_rot ? MV_GU_ROT : (p.direct ? MV_GU_DIRECT : MV_GU));
    // a directly routed token: the item count is known here, so no
    // workgroup is launched without an item
    const int direct_items = p.topk * ((p.n >> 7) / p.bx_per_item) * p.proj_launch * p.splits;
#define EXL3_MV_G(CBV, NSV, MVV, KWV, FXV, GFV)                                                        \
    if (cb == CBV && ns == NSV && mv == MVV && p.kw == KWV && fxs == FXV && gfx == GFV) {              \
        const void* fn = reinterpret_cast<const void*>(&moe_gemv_kernel<K, CBV, NSV, MVV, KWV, FXV, GFV>); \
        const int lrc = allow_dynamic_lds(fn, smem, "exl3 moe");                                       \
        if (lrc) return lrc;                                                                           \
        int grid = moe_grid_size(fn, threads, smem);                                                   \
        if (grid <= 0) return EXL3_ERR_HIP;                                                            \
        if (p.direct && grid > direct_items) grid = direct_items;                                      \
        moe_gemv_kernel<K, CBV, NSV, MVV, KWV, FXV, GFV><<<grid, threads, smem, st>>>(p);              \
        return launch_status("exl3 moe launch");                                                      \
    }
#define EXL3_MV_F(CBV, NSV, MVV, KWV, FXV) EXL3_MV_G(CBV, NSV, MVV, KWV, FXV, false)
#define EXL3_MV_KW(CBV, NSV, MVV, KWV) EXL3_MV_F(CBV, NSV, MVV, KWV, false)
#define EXL3_MV_NS(CBV, NSV, MVV) EXL3_MV_KW(CBV, NSV, MVV, 1) EXL3_MV_KW(CBV, NSV, MVV, 2)
#define EXL3_MV_MODES(CBV, NSV)                                                                        \
    EXL3_MV_NS(CBV, NSV, MV_GU) EXL3_MV_NS(CBV, NSV, MV_GU_ROT) EXL3_MV_NS(CBV, NSV, MV_DOWN)             \
    EXL3_MV_KW(CBV, NSV, MV_GU_DIRECT, 1) EXL3_MV_KW(CBV, NSV, MV_DOWN_DIRECT, 1)                        \
    EXL3_MV_F(CBV, NSV, MV_DOWN, 1, true) EXL3_MV_F(CBV, NSV, MV_DOWN_DIRECT, 1, true)
#define EXL3_MV_GFX(CBV, NSV)                                                                             \
    EXL3_MV_G(CBV, NSV, MV_GU_DIRECT, 1, true, true) EXL3_MV_G(CBV, NSV, MV_DOWN_DIRECT, 1, true, true)      \
    EXL3_MV_G(CBV, NSV, MV_GU_ROT, 1, true, true) EXL3_MV_G(CBV, NSV, MV_DOWN, 1, true, true)
#define EXL3_MV_CASE(CBV)                                                                                     \
    EXL3_MV_MODES(CBV, 2) EXL3_MV_MODES(CBV, 4) EXL3_MV_MODES(CBV, 8) EXL3_MV_MODES(CBV, 12) EXL3_MV_MODES(CBV, 16) \
    EXL3_MV_GFX(CBV, 2) EXL3_MV_GFX(CBV, 4) EXL3_MV_GFX(CBV, 8)
    EXL3_MV_CASE(0) EXL3_MV_CASE(1) EXL3_MV_CASE(2)
#undef EXL3_MV_CASE
#undef EXL3_MV_MODES
#undef EXL3_MV_GFX
#undef EXL3_MV_NS
#undef EXL3_MV_KW
#undef EXL3_MV_F
#undef EXL3_MV_G
    set_error("exl3 moe: no kernel for codebook %d steps %d k waves %d%s", cb, ns, p.kw,
              gfx ? " (split fixed-point gate/up)" : "");
    return EXL3_ERR_UNSUPPORTED;
}

// Workgroups of the fused one-token kernel that the device holds at once: the
// smaller of moe_grid_size's estimate and the runtime's occupancy figure
// (the fused launch relies on every workgroup being resident).
int moe_fused_grid_size(const void* fn, size_t smem);

// Step counts of the split fixed-point gate/up instances (and their down pass).
inline bool moe_gfx_steps_ok(int ns) { return ns == 2 || ns == 4 || ns == 8; }

// Step counts the fused one-token kernel is instantiated for (per pass).
inline bool moe_fused_steps_ok(int ns) { return ns == 2 || ns == 4 || ns == 8; }

// Step counts the fused routed kernel is instantiated for: gate/up, down
// (gfx: split fixed-point gate/up; dfx: split fixed-point down).
inline bool moe_fused_routed_steps_ok(int nsg, int nsd, bool gfx, bool dfx) {
    if (nsg != 8 || (gfx && !dfx)) return false;
    return nsd == 4 || nsd == 8 || (nsd == 12 && !gfx);
}

template <int K>
int moe_fused_launch_k(int cb, int nsg, int nsd, const MoeParams& pg, const MoeParams& pd, hipStream_t st) {
    const bool gfx = pg.gfx != 0;
    const size_t sg = moe_smem_bytes(4 * nsg, 1, gfx), sd = moe_smem_bytes(4 * nsd, 1, gfx);
    if (!pg.direct) {
        // routed batch: the item count is on the device, so the grid is the
        // resident capacity and workgroups past the items exit at once
        const bool dfx = pd.fxs != 0;
        const size_t sdr = moe_smem_bytes(4 * nsd, 1, dfx);
        const size_t smem = sg > sdr ? sg : sdr;
#define EXL3_MFR(CBV, NG, ND, GFV, DFV)                                                                     \
    if (cb == CBV && nsg == NG && nsd == ND && gfx == GFV && dfx == DFV) {                                 \
        const void* fn = reinterpret_cast<const void*>(&moe_fused_routed_kernel<K, CBV, NG, ND, GFV, DFV>); \
        const int lrc = allow_dynamic_lds(fn, smem, "exl3 moe fused routed");                              \
        if (lrc) return lrc;                                                                               \
        const int grid = moe_fused_grid_size(fn, smem);                                                    \
        if (grid <= 0) return EXL3_ERR_HIP;                                                                \
        moe_fused_routed_kernel<K, CBV, NG, ND, GFV, DFV><<<grid, 256, smem, st>>>(pg, pd);                \
        return launch_status("exl3 moe fused routed launch");                                              \
    }
#define EXL3_MFR_CB(CBV)                                                                                     \
    EXL3_MFR(CBV, 8, 8, false, false) EXL3_MFR(CBV, 8, 8, false, true) EXL3_MFR(CBV, 8, 12, false, false) \
    EXL3_MFR(CBV, 8, 12, false, true) EXL3_MFR(CBV, 8, 8, true, true) EXL3_MFR(CBV, 8, 4, false, true)    \
    EXL3_MFR(CBV, 8, 4, true, true) EXL3_MFR(CBV, 8, 4, false, false)
        EXL3_MFR_CB(0) EXL3_MFR_CB(1) EXL3_MFR_CB(2)
#undef EXL3_MFR_CB
#undef EXL3_MFR
        set_error("exl3 moe: no fused routed kernel for codebook %d steps %d / %d", cb, nsg, nsd);
        return EXL3_ERR_UNSUPPORTED;
    }
    const size_t smem = sg > sd ? sg : sd;
    const int items = pg.topk * ((pg.n >> 7) / pg.bx_per_item) * pg.proj_launch * pg.splits +
                      pd.topk * ((pd.n >> 7) / pd.bx_per_item) * pd.splits;
#define EXL3_MF(CBV, NG, ND, GFV)                                                                      \
    if (cb == CBV && nsg == NG && nsd == ND && gfx == GFV) {                                           \
        const void* fn = reinterpret_cast<const void*>(&moe_fused_direct_kernel<K, CBV, NG, ND, GFV>); \
        const int lrc = allow_dynamic_lds(fn, smem, "exl3 moe fused");                                 \
        if (lrc) return lrc;                                                                           \
        int grid = moe_fused_grid_size(fn, smem);                                                      \
        if (grid <= 0) return EXL3_ERR_HIP;                                                            \
        if (grid > items) grid = items;                                                                \
        moe_fused_direct_kernel<K, CBV, NG, ND, GFV><<<grid, 256, smem, st>>>(pg, pd);                 \
        return launch_status("exl3 moe fused launch");                                                 \
    }
#define EXL3_MF_G(CBV, NG)                                                                                    \
    EXL3_MF(CBV, NG, 2, false) EXL3_MF(CBV, NG, 4, false) EXL3_MF(CBV, NG, 8, false) EXL3_MF(CBV, NG, 2, true) \
    EXL3_MF(CBV, NG, 4, true) EXL3_MF(CBV, NG, 8, true)
#define EXL3_MF_CB(CBV) EXL3_MF_G(CBV, 2) EXL3_MF_G(CBV, 4) EXL3_MF_G(CBV, 8)
    EXL3_MF_CB(0) EXL3_MF_CB(1) EXL3_MF_CB(2)
#undef EXL3_MF_CB
#undef EXL3_MF_G
#undef EXL3_MF
    set_error("exl3 moe: no fused kernel for codebook %d steps %d / %d", cb, nsg, nsd);
    return EXL3_ERR_UNSUPPORTED;
}

// One instantiation unit per K (exl3_moe_inst.hip built with -DEXL3_K=K).
int moe_launch(int K, int cb, int ns, const MoeParams& p, hipStream_t st);
int moe_fused_launch(int K, int cb, int nsg, int nsd, const MoeParams& pg, const MoeParams& pd, hipStream_t st);

}  // namespace exl3
