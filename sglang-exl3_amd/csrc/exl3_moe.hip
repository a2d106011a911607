// C ABI of the batched MoE layer (exl3_moe_layer, exl3_p2b_fused_moe) and
// its launch planner.
#include <math.h>
#include <stdlib.h>

#include "exl3_moe_impl.h"

namespace exl3 {

int moe_launch_K1(int, int, int, const MoeParams&, dim3, hipStream_t);
int moe_launch_K2(int, int, int, const MoeParams&, dim3, hipStream_t);
int moe_launch_K3(int, int, int, const MoeParams&, dim3, hipStream_t);
int moe_launch_K4(int, int, int, const MoeParams&, dim3, hipStream_t);
int moe_launch_K5(int, int, int, const MoeParams&, dim3, hipStream_t);
int moe_launch_K6(int, int, int, const MoeParams&, dim3, hipStream_t);
int moe_launch_K7(int, int, int, const MoeParams&, dim3, hipStream_t);
int moe_launch_K8(int, int, int, const MoeParams&, dim3, hipStream_t);

int moe_launch(int K, int cb, int mb, int ns, const MoeParams& p, dim3 grid, hipStream_t st) {
    switch (K) {
        case 1: return moe_launch_K1(cb, mb, ns, p, grid, st);
        case 2: return moe_launch_K2(cb, mb, ns, p, grid, st);
        case 3: return moe_launch_K3(cb, mb, ns, p, grid, st);
        case 4: return moe_launch_K4(cb, mb, ns, p, grid, st);
        case 5: return moe_launch_K5(cb, mb, ns, p, grid, st);
        case 6: return moe_launch_K6(cb, mb, ns, p, grid, st);
        case 7: return moe_launch_K7(cb, mb, ns, p, grid, st);
        case 8: return moe_launch_K8(cb, mb, ns, p, grid, st);
    }
    set_error("exl3 moe: K=%d outside 1..8", K);
    return EXL3_ERR_UNSUPPORTED;
}

// ------------------------------------------------------------------ routing

// Group the entries by expert.  Entries with ids outside [0, E) are dropped.
// Row order inside an expert follows LDS atomics; each row's product is
// independent of its position, so results do not depend on it.
__global__ __launch_bounds__(MOE_ROUTE_THREADS) void moe_route_kernel(const int32_t* ids, int entries, int E,
                                                                     MoeRoute rt) {
    extern __shared__ __align__(16) int rt_smem[];
    int* cnt = rt_smem;        // [E]
    int* off = cnt + E;        // [E]
    int* rank = off + E;       // [E]
    int* pos = rank + E;       // [entries]
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += MOE_ROUTE_THREADS) cnt[e] = 0;
    __syncthreads();
    const EXL3_GLOBAL int32_t* idg = gptr(ids);
    for (int i = tid; i < entries; i += MOE_ROUTE_THREADS) {
        const int e = idg[i];
        pos[i] = (e >= 0 && e < E) ? atomicAdd(&cnt[e], 1) : -1;
    }
    __syncthreads();
    // exclusive scans of counts and of "active" over the experts, one wave
    if (tid < 64) {
        const int chunk = (E + 63) / 64;
        const int e0 = tid * chunk, e1 = min(E, e0 + chunk);
        int sr = 0, sa = 0;
        for (int e = e0; e < e1; ++e) {
            sr += cnt[e];
            sa += cnt[e] > 0;
        }
        int ir = sr, ia = sa;  // inclusive wave scan
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int pr = __shfl_up(ir, d), pa = __shfl_up(ia, d);
            if (tid >= d) {
                ir += pr;
                ia += pa;
            }
        }
        int r = ir - sr, a = ia - sa;
        for (int e = e0; e < e1; ++e) {
            off[e] = r;
            rank[e] = a;
            r += cnt[e];
            a += cnt[e] > 0;
        }
        if (tid == 63) gptr(rt.num_active)[0] = ia;
    }
    __syncthreads();
    for (int i = tid; i < entries; i += MOE_ROUTE_THREADS) {
        const int p = pos[i];
        if (p >= 0) gptr(rt.rows)[off[idg[i]] + p] = i;
    }
    for (int e = tid; e < E; e += MOE_ROUTE_THREADS) {
        const int c = cnt[e];
        if (c > 0) {
            const int a = rank[e];
            gptr(rt.act_expert)[a] = e;
            gptr(rt.act_off)[a] = off[e];
            gptr(rt.act_cnt)[a] = c;
        }
    }
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
    st_h2(gptr(out) + (size_t)t * hidden + c, __floats2half2_rn(a0, a1));
}

namespace {

constexpr int kMoeMaxExperts = 4096;
constexpr int kMoeMaxEntries = 8192;

struct MoePlan {
    int mb, ns, kw, splits;
};

int env_int(const char* name, int dflt) {
    const char* v = getenv(name);
    if (!v || !*v) return dflt;
    return atoi(v);
}

// Active experts expected for `tokens` tokens routed to `topk` of E experts
// uniformly: E (1 - (1 - topk/E)^tokens), capped by the slot count.
double expected_active(int tokens, int topk, int E) {
    const double u = (double)E * (1.0 - pow(1.0 - (double)topk / E, tokens));
    const double cap = (double)(E < tokens * topk ? E : tokens * topk);
    return u < cap ? u : cap;
}

// Same rule as the dense GEMV planner: the most work per wave that still puts
// `target` waves on the device, for the expected number of active experts.
MoePlan plan_moe(int rows_cap, int k, int n, int nproj, double active) {
    MoePlan pl{rows_cap <= 16 ? 1 : (rows_cap <= 32 ? 2 : 4), 0, 0, 0};
    const int kslices = k / 16;
    const long long target = env_int("EXL3_MOE_TARGET_WAVES", 3072);
    const int f_steps = env_int("EXL3_MOE_NSTEPS", 0), f_kw = env_int("EXL3_MOE_KW", 0);
    const double cols = (double)(n / 128) * nproj * active;
    MoePlan best = pl;
    double best_waves = -1;
    for (int kw = 2; kw >= 1; --kw) {
        for (int ns = 8; ns >= 2; ns /= 2) {
            const int kts_wg = 4 * ns * kw;
            if (kts_wg % 8 || kslices % kts_wg) continue;
            if (moe_smem_bytes(pl.mb, kts_wg, kw) > kMaxLds - 1024) continue;  // headroom for static LDS
            if ((f_steps && ns != f_steps) || (f_kw && kw != f_kw)) continue;
            const int S = kslices / kts_wg;
            const double waves = cols * S * 4 * kw;
            const bool better = waves >= target ? (best_waves < target || S < best.splits)
                                                : (best_waves < target && waves > best_waves);
            if (better) {
                best = MoePlan{pl.mb, ns, kw, S};
                best_waves = waves;
            }
        }
    }
    if (best.ns == 0) best = MoePlan{pl.mb, 2, 1, kslices / 8};
    return best;
}

struct MoeLayout {
    int slots, entries;
    MoePlan gu, dn;
    size_t route_off, h_off, y_off, part_off, total;
};

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

MoeLayout moe_layout(int tokens, int topk, int E, int hidden, int inter) {
    MoeLayout L{};
    L.entries = tokens * topk;
    L.slots = E < L.entries ? E : L.entries;
    const int rows_cap = tokens < 64 ? tokens : 64;
    const double act = expected_active(tokens, topk, E);
    L.gu = plan_moe(rows_cap, hidden, inter, 2, act);
    L.dn = plan_moe(rows_cap, inter, hidden, 1, act);
    size_t o = kWsCounterBytes;
    L.route_off = o;
    o = align256(o + (size_t)(1 + 3 * L.slots + L.entries) * sizeof(int));
    L.h_off = o;
    o = align256(o + (size_t)L.entries * inter * 2);
    L.y_off = o;
    o = align256(o + (size_t)L.entries * hidden * 2);
    L.part_off = o;
    const size_t pg = (size_t)(inter / 128) * 2 * L.gu.splits;
    const size_t pd = (size_t)(hidden / 128) * 1 * L.dn.splits;
    o = align256(o + (pg > pd ? pg : pd) * L.entries * 128 * sizeof(float));
    L.total = o;
    return L;
}

struct MoeTables {
    const int64_t *gt, *gs, *gv, *ut, *us, *uv, *dt, *ds, *dv;
};

int run_moe(const char* fn, const uint16_t* x, const int32_t* ids, const void* weights, int weights_f16,
            const MoeTables& tb, int E, uint16_t* out, int tokens, int topk, int hidden, int inter, int KG,
            int KU, int KD, int cb, float limit, void* ws, size_t ws_bytes, hipStream_t st) {
    EXL3_REQUIRE(tokens >= 1 && topk >= 1, "%s: tokens=%d topk=%d must be >= 1", fn, tokens, topk);
    EXL3_REQUIRE(E >= 1 && E <= kMoeMaxExperts, "%s: num_experts=%d outside 1..%d", fn, E, kMoeMaxExperts);
    EXL3_REQUIRE((long long)tokens * topk <= kMoeMaxEntries, "%s: tokens*topk=%lld above %d", fn,
                 (long long)tokens * topk, kMoeMaxEntries);
    EXL3_REQUIRE(hidden > 0 && inter > 0 && hidden % 128 == 0 && inter % 128 == 0,
                 "%s: hidden=%d inter=%d must be positive multiples of 128", fn, hidden, inter);
    EXL3_REQUIRE(KG >= 1 && KG <= 8 && KU >= 1 && KU <= 8 && KD >= 1 && KD <= 8,
                 "%s: K (gate %d, up %d, down %d) outside 1..8", fn, KG, KU, KD);
    EXL3_REQUIRE(cb >= 0 && cb <= 2, "%s: codebook=%d outside 0..2", fn, cb);
    EXL3_REQUIRE(x && ids && weights && out && tb.gt && tb.gs && tb.gv && tb.ut && tb.us && tb.uv && tb.dt &&
                     tb.ds && tb.dv,
                 "%s: null pointer", fn);
    EXL3_REQUIRE(aligned(x, 4) && aligned(out, 4), "%s: misaligned x/out", fn);
    const MoeLayout L = moe_layout(tokens, topk, E, hidden, inter);
    EXL3_REQUIRE_CODE(ws && ws_bytes >= L.total, EXL3_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, %zu given",
                      fn, L.total, ws ? ws_bytes : (size_t)0);
    const int nblk_max = (hidden > inter ? hidden : inter) / 128;
    EXL3_REQUIRE_CODE((size_t)L.slots * nblk_max <= kWsMaxCounters, EXL3_ERR_UNSUPPORTED,
                      "%s: %d slots x %d column blocks exceed the workspace counters", fn, L.slots, nblk_max);

    char* w8 = reinterpret_cast<char*>(ws);
    MoeRoute rt;
    int* ri = reinterpret_cast<int*>(w8 + L.route_off);
    rt.num_active = ri;
    rt.act_expert = ri + 1;
    rt.act_off = rt.act_expert + L.slots;
    rt.act_cnt = rt.act_off + L.slots;
    rt.rows = rt.act_cnt + L.slots;
    __half* h = reinterpret_cast<__half*>(w8 + L.h_off);
    __half* yslots = reinterpret_cast<__half*>(w8 + L.y_off);

    // 1. routing
    {
        const size_t smem = moe_route_smem_bytes(E, L.entries);
        int rc = allow_dynamic_lds(reinterpret_cast<const void*>(&moe_route_kernel), smem, "exl3 moe route");
        if (rc) return rc;
        moe_route_kernel<<<1, MOE_ROUTE_THREADS, smem, st>>>(ids, L.entries, E, rt);
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

    // 2. gate + up (+ SwiGLU + down input rotation)
    p.mode = MOE_GATE_UP;
    p.x = reinterpret_cast<const __half*>(x);
    p.t_tab0 = tb.gt;
    p.su_tab0 = tb.gs;
    p.sv_tab0 = tb.gv;
    p.t_tab1 = tb.ut;
    p.su_tab1 = tb.us;
    p.sv_tab1 = tb.uv;
    p.dsu_tab = tb.ds;
    p.out = h;
    p.k = hidden;
    p.n = inter;
    p.nproj = 2;
    p.splits = L.gu.splits;
    p.kw = L.gu.kw;
    int rc;
    if (KG == KU) {
        p.proj_base = 0;
        rc = moe_launch(KG, cb, L.gu.mb, L.gu.ns, p, dim3(inter / 128, 2 * L.gu.splits, L.slots), st);
        if (rc) return rc;
    } else {
        p.proj_base = 0;
        rc = moe_launch(KG, cb, L.gu.mb, L.gu.ns, p, dim3(inter / 128, L.gu.splits, L.slots), st);
        if (rc) return rc;
        p.proj_base = 1;
        rc = moe_launch(KU, cb, L.gu.mb, L.gu.ns, p, dim3(inter / 128, L.gu.splits, L.slots), st);
        if (rc) return rc;
    }

    // 3. down
    p.mode = MOE_DOWN;
    p.x = h;
    p.t_tab0 = tb.dt;
    p.su_tab0 = tb.ds;
    p.sv_tab0 = tb.dv;
    p.t_tab1 = p.su_tab1 = p.sv_tab1 = nullptr;
    p.dsu_tab = nullptr;
    p.out = yslots;
    p.k = inter;
    p.n = hidden;
    p.nproj = 1;
    p.proj_base = 0;
    p.splits = L.dn.splits;
    p.kw = L.dn.kw;
    rc = moe_launch(KD, cb, L.dn.mb, L.dn.ns, p, dim3(hidden / 128, L.dn.splits, L.slots), st);
    if (rc) return rc;

    // 4. weighted combine
    moe_combine_kernel<<<dim3((hidden / 2 + 255) / 256, tokens), 256, 0, st>>>(
        yslots, ids, weights, weights_f16, topk, E, hidden, reinterpret_cast<__half*>(out));
    return launch_status("exl3 moe combine launch");
}

}  // namespace
}  // namespace exl3

using namespace exl3;

extern "C" size_t exl3_moe_workspace_size(int tokens, int topk, int num_experts, int hidden, int inter) {
    if (tokens < 1 || topk < 1 || num_experts < 1 || hidden < 128 || inter < 128) return 0;
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
        out[4 * j + 0] = pls[j]->mb;
        out[4 * j + 1] = pls[j]->ns;
        out[4 * j + 2] = pls[j]->kw;
        out[4 * j + 3] = pls[j]->splits;
    }
    out[8] = L.slots;
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
    MoeTables tb{gate_trellis, gate_suh, gate_svh, up_trellis, up_suh, up_svh, down_trellis, down_suh, down_svh};
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
    MoeTables tb{gate_trellis, gate_suh, gate_svh, up_trellis, up_suh, up_svh, down_trellis, down_suh, down_svh};
    return run_moe("exl3_p2b_fused_moe", x, expert_ids, routing_weights, 1, tb, num_experts, out, 1, num_ids,
                   hidden, inter, K_gate, K_up, K_down, codebook, swiglu_limit, workspace, workspace_bytes,
                   as_stream(stream));
}
