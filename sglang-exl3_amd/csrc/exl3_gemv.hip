// C ABI of the GEMV family (exl3_gemv, exl3_gemm's skinny path,
// exl3_p2b_gemv_batched) and the gfx950 launch-shape selector that replaces
// the reference's per-architecture tables (csrc/exl3_gemv.cu:10-21, 40-48;
// csrc/quant/exl3_kernel_map.cuh:53-62).
#include <stdlib.h>

#include "exl3_gemv_sk.h"

namespace exl3 {

int gemv_launch_K1(int, int, const GemvParams&, int, hipStream_t);
int gemv_launch_K2(int, int, const GemvParams&, int, hipStream_t);
int gemv_launch_K3(int, int, const GemvParams&, int, hipStream_t);
int gemv_launch_K4(int, int, const GemvParams&, int, hipStream_t);
int gemv_launch_K5(int, int, const GemvParams&, int, hipStream_t);
int gemv_launch_K6(int, int, const GemvParams&, int, hipStream_t);
int gemv_launch_K7(int, int, const GemvParams&, int, hipStream_t);
int gemv_launch_K8(int, int, const GemvParams&, int, hipStream_t);

int gemv_sk_launch_K1(int, int, const GemvSkParams&, hipStream_t);
int gemv_sk_launch_K2(int, int, const GemvSkParams&, hipStream_t);
int gemv_sk_launch_K3(int, int, const GemvSkParams&, hipStream_t);
int gemv_sk_launch_K4(int, int, const GemvSkParams&, hipStream_t);
int gemv_sk_launch_K5(int, int, const GemvSkParams&, hipStream_t);
int gemv_sk_launch_K6(int, int, const GemvSkParams&, hipStream_t);
int gemv_sk_launch_K7(int, int, const GemvSkParams&, hipStream_t);
int gemv_sk_launch_K8(int, int, const GemvSkParams&, hipStream_t);

int gemv_sk_launch(int K, int cb, int ns, const GemvSkParams& p, hipStream_t st) {
    switch (K) {
        case 1: return gemv_sk_launch_K1(cb, ns, p, st);
        case 2: return gemv_sk_launch_K2(cb, ns, p, st);
        case 3: return gemv_sk_launch_K3(cb, ns, p, st);
        case 4: return gemv_sk_launch_K4(cb, ns, p, st);
        case 5: return gemv_sk_launch_K5(cb, ns, p, st);
        case 6: return gemv_sk_launch_K6(cb, ns, p, st);
        case 7: return gemv_sk_launch_K7(cb, ns, p, st);
        case 8: return gemv_sk_launch_K8(cb, ns, p, st);
    }
    set_error("exl3 gemv: K=%d outside 1..8", K);
    return EXL3_ERR_UNSUPPORTED;
}

int gemv_launch(int K, int cb, int mb, const GemvParams& p, int experts, hipStream_t st) {
    switch (K) {
        case 1: return gemv_launch_K1(cb, mb, p, experts, st);
        case 2: return gemv_launch_K2(cb, mb, p, experts, st);
        case 3: return gemv_launch_K3(cb, mb, p, experts, st);
        case 4: return gemv_launch_K4(cb, mb, p, experts, st);
        case 5: return gemv_launch_K5(cb, mb, p, experts, st);
        case 6: return gemv_launch_K6(cb, mb, p, experts, st);
        case 7: return gemv_launch_K7(cb, mb, p, experts, st);
        case 8: return gemv_launch_K8(cb, mb, p, experts, st);
    }
    set_error("exl3 gemv: K=%d outside 1..8", K);
    return EXL3_ERR_UNSUPPORTED;
}

int fat_gemm_rows(const uint16_t* x, const int16_t* trellis, const uint16_t* suh, const uint16_t* svh, uint16_t* y,
                  int m, int k, int n, int K, int cb, void* ws, size_t ws_bytes, hipStream_t st);

// Rows up to which exl3_gemm runs the GEMV kernels; above, the input is
// rotated once and the MFMA GEMM runs (env EXL3_GEMM_GEMV_ROWS, at most 64).
// The MFMA path parallelises over 128-column blocks, so it wins earlier on
// wide outputs.  Graph-timed, GEMV / MFMA (split hand-off), K = 3 unless
// noted: k = 4096, n = 7168: m = 8 / 12 / 16: 13.6 / 16.2 / 18.4 against 15.7 /
// 16.7 / 17.3 us; k = 14336, n = 4096: m = 8 / 12 / 16: 18.8 / 24.1 / 32.6
// against 23.9 / 25.2 / 26.8; k = 4096, n = 14336, K = 4: m = 8 / 9 / 12: 18.7 /
// 20.0 / 22.9 against 18.7 / 19.5 / 19.9; k = 4096, n = 28672: m = 4 / 8: 23.7
// / 30.9 against 27.6 / 28.3.
int gemm_gemv_rows(int n) {
    const char* v = getenv("EXL3_GEMM_GEMV_ROWS");
    const int r = (v && *v) ? atoi(v) : (n >= 24576 ? kGemmGemvRowsWide - 1
                                                    : (n >= 12288 ? kGemmGemvRowsWide : kGemmGemvRows));
    return r < 0 ? 0 : (r > 64 ? 64 : r);
}

namespace {

constexpr int kMaxGemvRows = 64;
constexpr size_t kMaxGemvSmem = kMaxLds - 1024;  // headroom for static LDS

struct GemvPlan {
    int mb;
    int nsteps;  // steps of 4 k-slices per wave
    int kw;      // k waves per workgroup
    int splits;  // workgroups along k
    int sk;      // 1: balanced kernel (gemv_sk_kernel, m <= 4): splits = pieces per column block, nsteps = piece length
};

// gfx950 launch shape.  Every workgroup covers one 128-column block (one
// output FWHT block) with 4 column waves, times kw k-waves, each walking
// `nsteps` steps of 4 k-slices.  Walk from the most work per wave to the least
// and take the first shape that puts at least `target` waves on the device
// (1024 SIMDs: ~3 waves each hide HBM and MFMA latency); this also keeps the
// number of cross-workgroup k-splits (the costly reduction) minimal.
// Balanced kernel shape (m <= 4): P equal pieces per 128-column block, P a
// divisor of k/64 with an instantiated piece length.  Cost model fitted to
// graph-timed sweeps on MI355X (k x n from 2048 x 6144 to 14336 x 4096):
// with W = ceil(workgroups / CUs) workgroups on the busiest CU and `steps`
// k-steps on it,
//   time ~ 0.242 us * steps + 0.089 us * W + 0.902 us / min(W, 4)
// (per-step work, per-workgroup overhead, and the latency that fewer than
// four workgroups per CU leave exposed).  Above kSkMaxRows rows the k-split
// kernel is used: the balanced kernel's per-workgroup input rotation and
// epilogue grow with m, and a variant fed by a separate row-rotation pass
// was slower too at every piece count (config 2, m = 2 / 8: 14.7 / 23.4 us
// against 13.7 / 20.1 us; the extra launch and the m x n x P fixed-point adds
// outweigh the balance).  Returns false when the balanced kernel does not
// apply.
// Rows up to which the balanced kernel is used (env EXL3_GEMV_SK_ROWS, up to
// 4).  Against the k-split kernel on config 2 (same run): m = 2: 11.5 ->
// 11.5 us; m = 3: 14.8 -> 14.0 us; m = 4: 15.2 -> 16.4 us (each row adds its
// input rotation to every workgroup and an epilogue wave).
constexpr int kSkMaxRows = 3;
constexpr int kSkInstRows = 4;

bool plan_gemv_sk(int m, int k, int n, int experts, int* ns_out, int* p_out) {
    const int max_rows = env_int("EXL3_GEMV_SK_ROWS", kSkMaxRows);
    if (experts != 1 || m > (max_rows < kSkInstRows ? max_rows : kSkInstRows) || env_int("EXL3_GEMV_SK", 1) == 0)
        return false;
    if ((size_t)m * n * 8 > kWsAccBytes) return false;
    const int ks_blk = k / 64;
    const long long nblk = n / 128;
    const int forced = env_int("EXL3_GEMV_SK_P", 0);
    const long long cus = 256;
    double best_cost = 1e30;
    bool found = false;
    for (int P = 1; P <= ks_blk && P <= SK_MAX_CONTRIB; ++P) {
        if (ks_blk % P || (forced && P != forced)) continue;
        const int ns = ks_blk / P;
        bool inst = false;
        for (int c : kSkSteps) inst |= c == ns;
        if (!inst || gemv_sk_smem_bytes(ns, gemv_sk_rows(m)) > kMaxGemvSmem) continue;
        const long long W = (nblk * P + cus - 1) / cus;
        const double cost = 0.242 * (double)(W * ns) + 0.089 * (double)W + 0.902 / (double)(W < 4 ? W : 4);
        if (cost < best_cost - 1e-9) {
            best_cost = cost;
            *ns_out = ns;
            *p_out = P;
            found = true;
        }
    }
    return found;
}

GemvPlan plan_gemv(int m, int k, int n, int K, int experts) {
    GemvPlan pl;
    int sk_ns = 0, sk_p = 0;
    if (plan_gemv_sk(m, k, n, experts, &sk_ns, &sk_p)) return GemvPlan{1, sk_ns, 1, sk_p, 1};
    pl.mb = m <= 16 ? 1 : (m <= 32 ? 2 : 4);
    const int kslices = k / 16;
    const int max_steps = 16;
    const long long target = env_int("EXL3_GEMV_TARGET_WAVES", 3072);
    const int f_steps = env_int("EXL3_GEMV_NSTEPS", 0), f_kw = env_int("EXL3_GEMV_KW", 0);
    const long long cols = (long long)(n / 128) * experts;
    GemvPlan best{pl.mb, 0, 0, 0, 0};
    long long best_waves = -1;
    for (int kw = 2; kw >= 1; --kw) {
        for (int ns = max_steps; ns >= 2; ns /= 2) {  // instantiated step counts: 16, 8, 4, 2
            const int kts_wg = 4 * ns * kw;
            if (kts_wg % 8 || kslices % kts_wg) continue;
            if (gemv_smem_bytes(m, kts_wg, kw) > kMaxGemvSmem) continue;
            if ((f_steps && ns != f_steps) || (f_kw && kw != f_kw)) continue;
            const int S = kslices / kts_wg;
            const long long waves = cols * S * 4 * kw;
            if (waves >= target) {
                if (best_waves < target || S < best.splits) {
                    best = GemvPlan{pl.mb, ns, kw, S, 0};
                    best_waves = waves;
                }
            } else if (best_waves < target && waves > best_waves) {
                best = GemvPlan{pl.mb, ns, kw, S, 0};
                best_waves = waves;
            }
        }
    }
    if (best.nsteps == 0) best = GemvPlan{pl.mb, 2, 1, kslices / 8, 0};  // 128-row ranges always fit
    return best;
}

// Rows from which a single-matrix k-split GEMV rotates its input once, in a
// launch of its own, instead of in every workgroup (each workgroup rotates
// every row of its k range).  Config 2, per-workgroup against separate
// rotation: m = 4: 15.4 / 16.4 us, 8: 19.0 / 19.8, 16: 30.6 / 30.3, 32: 62.2 /
// 57.8, 64: 126.9 / 116.2 (the launch costs ~1 us).  Env EXL3_GEMV_ROT_ROWS
// overrides (0: never).
constexpr int kGemvRotRows = 32;

bool gemv_pre_rotates(const GemvPlan& pl, int m, int experts) {
    const int rows = env_int("EXL3_GEMV_ROT_ROWS", kGemvRotRows);
    return !pl.sk && experts == 1 && rows > 0 && m >= rows;
}

// k-split hand-off of a single-matrix call through the fixed-point
// accumulators (one round trip: every split rotates and adds its own partial
// rows; gemv_kernel<.., FX = true>) instead of partial tiles, a counter and
// a last arrival that sums them (three round trips).  Every split then pays
// the output rotation and m x 128 adds per column block, so it pays off for
// few rows only.  Config 2 graph-timed, fixed-point vs partials: m = 4 / 8 /
// 12 / 16 / 32: 14.5 / 18.8-19.0 / 24.7 / 34.0 / 77.0 us vs 15.5 / 19.1 /
// 22.8 / 30.9 / 58.1 us.  Env EXL3_GEMV_FX_ROWS overrides the row limit
// (0: never).
constexpr int kGemvFxRows = 8;

bool gemv_fx(const GemvPlan& pl, int m, int n, int experts) {
    return !pl.sk && experts == 1 && pl.splits > 1 && pl.splits <= SK_MAX_CONTRIB && m <= 32 &&
           m <= env_int("EXL3_GEMV_FX_ROWS", kGemvFxRows) && (size_t)m * n * 8 <= kWsAccBytes;
}

// Workspace: [counters][accumulators][partials (k-split without the
// fixed-point hand-off), then the rotated rows (pre-rotating calls)].
size_t gemv_partials_bytes(const GemvPlan& pl, int m, int n, int experts) {
    if (pl.splits <= 1 || gemv_fx(pl, m, n, experts)) return 0;
    return (((size_t)(n / 128) * experts * pl.splits * (size_t)m * 128 * sizeof(float)) + 255) & ~(size_t)255;
}

size_t workspace_bytes_for(const GemvPlan& pl, int m, int k, int n, int experts) {
    if (pl.sk) return kWsAccOffset + (size_t)m * n * 8;
    const size_t part = gemv_partials_bytes(pl, m, n, experts);
    const size_t xr = gemv_pre_rotates(pl, m, experts) ? (size_t)m * k * 2 : 0;
    if (part == 0 && xr == 0) return gemv_fx(pl, m, n, experts) ? kWsAccOffset + (size_t)m * n * 8 : 0;
    return kWsScratchOffset + part + xr;
}

int check_common(const char* fn, int m, int k, int n, int K, int codebook) {
    EXL3_REQUIRE(m >= 1, "%s: m=%d must be >= 1", fn, m);
    EXL3_REQUIRE(k > 0 && n > 0 && k % 128 == 0 && n % 128 == 0,
                 "%s: k=%d n=%d must be positive multiples of 128", fn, k, n);
    EXL3_REQUIRE(K >= 1 && K <= 8, "%s: K=%d outside 1..8", fn, K);
    EXL3_REQUIRE(codebook >= 0 && codebook <= 2, "%s: codebook=%d outside 0..2", fn, codebook);
    return EXL3_OK;
}

int run_gemv(const char* fn, GemvParams p, int K, int codebook, int experts, void* ws, size_t ws_bytes,
             hipStream_t st) {
    GemvPlan pl = plan_gemv(p.m, p.k, p.n, K, experts);
    const size_t need = workspace_bytes_for(pl, p.m, p.k, p.n, experts);
    EXL3_REQUIRE_CODE(need == 0 || (ws && ws_bytes >= need), EXL3_ERR_WORKSPACE,
                      "%s: workspace of %zu bytes needed, %zu given", fn, need, ws ? ws_bytes : (size_t)0);
    if (pl.sk) {
        GemvSkParams q{};
        q.x = p.x;
        q.trellis = p.trellis;
        q.suh = p.suh;
        q.svh = p.svh;
        q.y = p.y;
        q.acc = reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(ws) + kWsAccOffset);
        q.m = p.m;
        q.k = p.k;
        q.n = p.n;
        q.pieces = pl.splits;
        return gemv_sk_launch(K, codebook, pl.nsteps, q, st);
    }
    p.nsteps = pl.nsteps;
    p.kw = pl.kw;
    p.splits = pl.splits;
    if (gemv_fx(pl, p.m, p.n, experts) && !p.gu) {
        p.fx = 1;
        p.acc = reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(ws) + kWsAccOffset);
    }
    if (need) {
        EXL3_REQUIRE_CODE((size_t)(p.n / 128) * experts <= kWsMaxCounters, EXL3_ERR_UNSUPPORTED,
                          "%s: %d column blocks exceed the %zu workspace counters", fn, (p.n / 128) * experts,
                          kWsMaxCounters);
        p.counters = reinterpret_cast<int*>(ws);
        p.partials = reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + kWsScratchOffset);
    } else {
        p.counters = nullptr;
        p.partials = nullptr;
    }
    if (gemv_pre_rotates(pl, p.m, experts) && !p.gu) {
        __half* xr = reinterpret_cast<__half*>(reinterpret_cast<char*>(ws) + kWsScratchOffset +
                                               gemv_partials_bytes(pl, p.m, p.n, experts));
        const long long chunks = (long long)p.m * (p.k / 128);
        rotate_rows_kernel<<<(unsigned)((chunks + 3) / 4), 256, 0, st>>>(p.x, p.suh, xr, chunks, p.k);
        const int rc = launch_status("exl3 gemv rotate launch");
        if (rc) return rc;
        p.x = xr;
        p.x_rot = 1;
    }
    return gemv_launch(K, codebook, pl.mb, p, experts, st);
}

GemvParams base_params(const uint16_t* x, const int16_t* trellis, const uint16_t* suh, const uint16_t* svh,
                       uint16_t* y, int m, int k, int n) {
    GemvParams p{};
    p.x = reinterpret_cast<const __half*>(x);
    p.trellis = reinterpret_cast<const uint32_t*>(trellis);
    p.suh = reinterpret_cast<const __half*>(suh);
    p.svh = reinterpret_cast<const __half*>(svh);
    p.y = reinterpret_cast<__half*>(y);
    p.m = m;
    p.k = k;
    p.n = n;
    return p;
}

// ----------------------------- dense gate + up on the GEMV kernel (m <= 64)

// Gate and up as the two "experts" of one k-split GEMV launch; the last of a
// column block's 2 S workgroups applies the SwiGLU.  Scratch: counters (one
// per column block) and the partials of both projections, always (the
// hand-off needs them even when the plan has a single split).
GemvPlan plan_gate_up(int m, int k, int n, int K) { return plan_gemv(m, k, n, K, 2); }

size_t gate_up_gemv_bytes(int m, int k, int n, int K) {
    const GemvPlan pl = plan_gate_up(m, k, n, K);
    return kWsScratchOffset + (size_t)2 * (n / 128) * pl.splits * (size_t)m * 128 * sizeof(float);
}

int run_gate_up_gemv(const uint16_t* x, const uint16_t* suh, const int16_t* gt, const uint16_t* gsv,
                     const int16_t* ut, const uint16_t* usv, uint16_t* out, int m, int k, int n, int K, int cb,
                     float limit, void* ws, size_t ws_bytes, hipStream_t st) {
    EXL3_REQUIRE_CODE(m <= 16, EXL3_ERR_UNSUPPORTED, "exl3_gate_up_swiglu: the GEMV path takes at most 16 rows, not %d",
                      m);
    const GemvPlan pl = plan_gate_up(m, k, n, K);
    const size_t need = gate_up_gemv_bytes(m, k, n, K);
    EXL3_REQUIRE_CODE(ws && ws_bytes >= need, EXL3_ERR_WORKSPACE,
                      "exl3_gate_up_swiglu: workspace of %zu bytes needed, %zu given", need, ws ? ws_bytes : (size_t)0);
    EXL3_REQUIRE_CODE((size_t)(n / 128) <= kWsMaxCounters, EXL3_ERR_UNSUPPORTED,
                      "exl3_gate_up_swiglu: %d column blocks exceed the workspace counters", n / 128);
    EXL3_REQUIRE(aligned(gt, 16) && aligned(ut, 16) && aligned(gsv, 4) && aligned(usv, 4),
                 "exl3_gate_up_swiglu: misaligned pointer");
    GemvParams p = base_params(x, gt, suh, gsv, out, m, k, n);
    p.gu = 1;
    p.trellis2 = reinterpret_cast<const uint32_t*>(ut);
    p.suh2 = reinterpret_cast<const __half*>(suh);
    p.svh2 = reinterpret_cast<const __half*>(usv);
    p.limit = limit;
    p.nsteps = pl.nsteps;
    p.kw = pl.kw;
    p.splits = pl.splits;
    p.counters = reinterpret_cast<int*>(ws);
    p.partials = reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + kWsScratchOffset);
    return gemv_launch(K, cb, pl.mb, p, 2, st);
}

}  // namespace

// Rows up to which exl3_gate_up_swiglu runs the GEMV kernel; above, the input
// is rotated once and the MFMA kernels run in gate/up mode.  Graph-timed on
// config 3 (k = 4096, n = 2 x 14336, K = 3), GEMV / MFMA: m = 1 / 2 / 3 / 4 /
// 8: 21.1 / 22.9 / 24.4-24.5 / 26.4 / 27.4 us against 24.5-25.3 / 24.9-25.1 /
// 24.8-25.1 / 25.1-25.5 / 27.1 us (the GEMV workgroups each re-rotate all m
// input rows of their k range).
constexpr int kGateUpMaxGemvRows = 3;
// The gate/up GEMV mode is instantiated for one MFMA row block only.
constexpr int kGateUpGemvRowLimit = 16;

// Rows up to which exl3_gate_up_swiglu takes the GEMV path: the default, or
// env EXL3_GATE_UP_GEMV_ROWS clamped to [0, kGateUpGemvRowLimit].
int gate_up_gemv_rows() {
    const int r = env_int("EXL3_GATE_UP_GEMV_ROWS", kGateUpMaxGemvRows);
    return r < 0 ? 0 : (r > kGateUpGemvRowLimit ? kGateUpGemvRowLimit : r);
}

size_t fat_gate_up_scratch_bytes(int m, int k, int n);
int fat_gate_up_rows(const uint16_t* x, const uint16_t* suh, const int16_t* gate_trellis, const uint16_t* gate_svh,
                     const int16_t* up_trellis, const uint16_t* up_svh, uint16_t* out, int m, int k, int n, int K,
                     int cb, float limit, void* ws, size_t ws_bytes, hipStream_t st);

}  // namespace exl3

using namespace exl3;

extern "C" size_t exl3_gate_up_workspace_size(int m, int k, int n, int K) {
    if (m < 1 || k < 128 || n < 128 || k % 128 || n % 128 || K < 1 || K > 8) return 0;
    const int gemv_rows = gate_up_gemv_rows();
    size_t need = m > gemv_rows ? fat_gate_up_scratch_bytes(m, k, n) : gate_up_gemv_bytes(m, k, n, K);
    if (m <= 64) {  // room for both paths (EXL3_GATE_UP_GEMV_ROWS moves the switch point)
        const size_t c = fat_gate_up_scratch_bytes(m, k, n), d = gate_up_gemv_bytes(m, k, n, K);
        need = need > c ? need : c;
        need = need > d ? need : d;
    }
    return need;
}

extern "C" int exl3_gate_up_swiglu(const uint16_t* x, const uint16_t* suh, const int16_t* gate_trellis,
                                   const uint16_t* gate_svh, const int16_t* up_trellis, const uint16_t* up_svh,
                                   uint16_t* out, int m, int k, int n, int K, int codebook, float swiglu_limit,
                                   void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    EXL3_REQUIRE(m >= 1, "exl3_gate_up_swiglu: m=%d must be >= 1", m);
    int rc = check_common("exl3_gate_up_swiglu", m, k, n, K, codebook);
    if (rc) return rc;
    EXL3_REQUIRE(x && suh && gate_trellis && gate_svh && up_trellis && up_svh && out,
                 "exl3_gate_up_swiglu: null pointer");
    EXL3_REQUIRE(aligned(x, 4) && aligned(out, 4) && aligned(suh, 4), "exl3_gate_up_swiglu: misaligned pointer");
    EXL3_REQUIRE(!(swiglu_limit < 0.0f) && swiglu_limit == swiglu_limit,
                 "exl3_gate_up_swiglu: swiglu_limit must be >= 0 (0 or inf: no clamp)");
    hipStream_t st = as_stream(stream);
    if (m > gate_up_gemv_rows())
        return fat_gate_up_rows(x, suh, gate_trellis, gate_svh, up_trellis, up_svh, out, m, k, n, K, codebook,
                                swiglu_limit, workspace, workspace_bytes, st);
    return run_gate_up_gemv(x, suh, gate_trellis, gate_svh, up_trellis, up_svh, out, m, k, n, K, codebook,
                            swiglu_limit, workspace, workspace_bytes, st);
}

extern "C" size_t exl3_gemv_workspace_size(int m, int k, int n, int K, int experts) {
    if (m < 1 || k < 128 || n < 128 || experts < 1) return 0;
    const int mc = m > kMaxGemvRows ? kMaxGemvRows : m;
    GemvPlan pl = plan_gemv(mc, k, n, K, experts);
    return workspace_bytes_for(pl, mc, k, n, experts);
}

extern "C" int exl3_gemv_plan(int m, int k, int n, int K, int experts, int* out) {
    clear_error();
    EXL3_REQUIRE(out, "exl3_gemv_plan: null pointer");
    int rc = check_common("exl3_gemv_plan", m > kMaxGemvRows ? kMaxGemvRows : m, k, n, K, 1);
    if (rc) return rc;
    const int mc = m > kMaxGemvRows ? kMaxGemvRows : m;
    GemvPlan pl = plan_gemv(mc, k, n, K, experts);
    out[0] = pl.mb;
    out[1] = pl.nsteps;
    out[2] = pl.kw;
    out[3] = pl.splits;
    out[4] = (int)(pl.sk ? gemv_sk_smem_bytes(pl.nsteps, gemv_sk_rows(m)) : gemv_smem_bytes(mc, 4 * pl.nsteps * pl.kw, pl.kw));
    return EXL3_OK;
}

extern "C" int exl3_gemv(const uint16_t* x, const int16_t* trellis, const uint16_t* suh, const uint16_t* svh,
                         uint16_t* y, int m, int k, int n, int K, int codebook, void* workspace,
                         size_t workspace_bytes, void* stream) {
    clear_error();
    int rc = check_common("exl3_gemv", m, k, n, K, codebook);
    if (rc) return rc;
    EXL3_REQUIRE(m <= kMaxGemvRows, "exl3_gemv: m=%d above %d (use exl3_gemm)", m, kMaxGemvRows);
    EXL3_REQUIRE(x && trellis && suh && svh && y, "exl3_gemv: null pointer");
    EXL3_REQUIRE(aligned(x, 4) && aligned(y, 4) && aligned(suh, 4) && aligned(svh, 4) && aligned(trellis, 16),
                 "exl3_gemv: misaligned pointer");
    GemvParams p = base_params(x, trellis, suh, svh, y, m, k, n);
    return run_gemv("exl3_gemv", p, K, codebook, 1, workspace, workspace_bytes, as_stream(stream));
}

extern "C" int exl3_gemm(const uint16_t* x, const int16_t* trellis, const uint16_t* suh, const uint16_t* svh,
                         uint16_t* y, int m, int k, int n, int K, int codebook, void* workspace,
                         size_t workspace_bytes, void* stream) {
    clear_error();
    int rc = check_common("exl3_gemm", m, k, n, K, codebook);
    if (rc) return rc;
    EXL3_REQUIRE(x && trellis && suh && svh && y, "exl3_gemm: null pointer");
    EXL3_REQUIRE(aligned(x, 4) && aligned(y, 4) && aligned(suh, 4) && aligned(svh, 4) && aligned(trellis, 16),
                 "exl3_gemm: misaligned pointer");
    hipStream_t st = as_stream(stream);
    if (m > gemm_gemv_rows(n)) return fat_gemm_rows(x, trellis, suh, svh, y, m, k, n, K, codebook, workspace,
                                               workspace_bytes, st);
    for (int r0 = 0; r0 < m; r0 += kMaxGemvRows) {
        const int mc = (m - r0) < kMaxGemvRows ? (m - r0) : kMaxGemvRows;
        GemvParams p = base_params(x + (size_t)r0 * k, trellis, suh, svh, y + (size_t)r0 * n, mc, k, n);
        rc = run_gemv("exl3_gemm", p, K, codebook, 1, workspace, workspace_bytes, st);
        if (rc) return rc;
    }
    return EXL3_OK;
}

extern "C" int exl3_p2b_gemv_batched(const uint16_t* x, int x_per_expert, const int64_t* trellis_ptrs,
                                     const int64_t* suh_ptrs, const int64_t* svh_ptrs, const int32_t* ids,
                                     int num_active, uint16_t* out, int m, int k, int n, int K, int codebook,
                                     void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    int rc = check_common("exl3_p2b_gemv_batched", m, k, n, K, codebook);
    if (rc) return rc;
    EXL3_REQUIRE(m <= kMaxGemvRows, "exl3_p2b_gemv_batched: m=%d above %d", m, kMaxGemvRows);
    EXL3_REQUIRE(num_active >= 1 && num_active <= 65535, "exl3_p2b_gemv_batched: num_active=%d", num_active);
    EXL3_REQUIRE(x && trellis_ptrs && suh_ptrs && svh_ptrs && ids && out, "exl3_p2b_gemv_batched: null pointer");
    GemvParams p = base_params(x, nullptr, nullptr, nullptr, out, m, k, n);
    p.t_tab = trellis_ptrs;
    p.su_tab = suh_ptrs;
    p.sv_tab = svh_ptrs;
    p.ids = ids;
    p.x_stride_e = x_per_expert ? (long long)m * k : 0;
    p.y_stride_e = (long long)m * n;
    return run_gemv("exl3_p2b_gemv_batched", p, K, codebook, num_active, workspace, workspace_bytes,
                    as_stream(stream));
}
