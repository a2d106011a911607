// C ABI of the many-row EXL3 GEMM: exl3_fat_gemm, exl3_fat_gemm_scatter and
// the prefill path of exl3_gemm (rotate -> fat GEMM -> fp16), with the launch
// planner (rows per tile, k-splits).
#include "exl3_fat_impl.h"

namespace exl3 {

int fat_launch_K1(int, int, const FatParams&, int, hipStream_t);
int fat_launch_K2(int, int, const FatParams&, int, hipStream_t);
int fat_launch_K3(int, int, const FatParams&, int, hipStream_t);
int fat_launch_K4(int, int, const FatParams&, int, hipStream_t);
int fat_launch_K5(int, int, const FatParams&, int, hipStream_t);
int fat_launch_K6(int, int, const FatParams&, int, hipStream_t);
int fat_launch_K7(int, int, const FatParams&, int, hipStream_t);
int fat_launch_K8(int, int, const FatParams&, int, hipStream_t);

int fat_launch(int K, int cb, int mt, const FatParams& p, int splits, hipStream_t st) {
    switch (K) {
        case 1: return fat_launch_K1(cb, mt, p, splits, st);
        case 2: return fat_launch_K2(cb, mt, p, splits, st);
        case 3: return fat_launch_K3(cb, mt, p, splits, st);
        case 4: return fat_launch_K4(cb, mt, p, splits, st);
        case 5: return fat_launch_K5(cb, mt, p, splits, st);
        case 6: return fat_launch_K6(cb, mt, p, splits, st);
        case 7: return fat_launch_K7(cb, mt, p, splits, st);
        case 8: return fat_launch_K8(cb, mt, p, splits, st);
    }
    set_error("exl3 fat gemm: K=%d outside 1..8", K);
    return EXL3_ERR_UNSUPPORTED;
}

namespace {

__global__ void fill_f32_kernel(float* p, size_t n, float v) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = v;
}

__global__ void f32_to_f16_kernel(const float* src, __half* dst, size_t n2) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n2; i += (size_t)gridDim.x * blockDim.x) {
        const float2 v = reinterpret_cast<const float2*>(src)[i];
        reinterpret_cast<__half2*>(dst)[i] = __floats2half2_rn(v.x, v.y);
    }
}

struct FatPlan {
    int mt, splits;
};

// Wide tiles (256 x 256, fat_big_kernel) above kFatNarrowMaxRows rows (env
// EXL3_FAT_WIDE=0 turns them off); up to there the narrow kernel with 16-row
// tiles up to 16 rows and 64-row tiles above.  k-splits for the narrow kernel
// up to kFatNarrowWgs workgroups (each split a whole number of FAT_CH
// chunks).  The wide kernel splits only grids under 96
// workgroups (an even number of steps per split): its outputs are large, and
// split outputs cost a zero fill plus one fp32 atomic per value and split,
// which measured slower than leaving up to 60 % of the CUs idle.
// Config 2 (n = 14336), graph-timed: 64-row narrow tiles / 128-row narrow
// tiles / wide tiles: M = 128: 68.7 / 108.8 / 99.0 us, 192: 78.0 / 109.6 /
// 111.7, 256: 81.0 / 110.7 / 125.3, 320: 128.8 / 172.0 / 126.8, 512: 154.8 /
// 222.6 / 129.6, 768: 227.9 / 330.7 / 131.4.  128-row narrow tiles never win
// (kept as the EXL3_FAT_MT=128 override).
constexpr int kFatNarrowMaxRows = 256;
// ... and only when they make at least this many tiles: a smaller wide grid
// needs fp32-atomic k-splits, and the narrow kernel with its split hand-off
// is faster there.  Graph-timed, wide / narrow: k = 14336, n = 4096, M = 320 /
// 512 / 768 / 1024 / 1536 / 2048 (20 / 32 / 48 / 64 / 96 / 128 tiles): 153.0 /
// 171.0 / 258.1 / 273.4 / 240.0 / 269.6 us against 101.4 / 129.9 / 191.9 /
// 241.3 / 361.0 / 458.5; k = 4096, n = 7168, M = 768 / 1024 (84 / 112 tiles):
// 151.0 / 99.0 against 105.6 / 131.1; n = 14336, M = 320 (112 tiles): 91.7
// against 97.0.
constexpr int kFatWideMinTiles = 96;

// k-splits of the narrow kernel: the most that keep the grid at or under
// kFatNarrowWgs workgroups (about two per CU; more splits add partial sums
// and shorten each workgroup's decode below what hides its latency).
// exl3_gemm, k = 4096, K = 4, graph-timed, splits 1 / 2 / 4 / 8: n = 14336,
// M = 16: 40.1 / 29.5 / 24.6 / 29.6 us, M = 64: 68.0 / 53.0 / 49.8 / 71.8,
// M = 128: 69.0 / 67.5 / 89.1 / 130.0; n = 28672, M = 16: 40.2 / 37.5 / 39.6 /
// 45.4, M = 128: 80.1 / 123.1 / 161.3 / 234.5.  (Gate/up mode has its own rule,
// plan_gate_up_fat.)
constexpr long long kFatNarrowWgs = 512;
// With fp16 output the splits hand partial tiles to the last split
// (fat_handoff), which costs less than the atomics: the most splits that keep
// the grid at or under kFatHandoffWgs workgroups (about the resident count)
// with at least kFatHandoffMinSteps steps per split.  Graph-timed, splits
// 1 / 2 / 4 / 8 / 16 with the hand-off: k = 4096, n = 14336, K = 4: M = 16:
// 37.3 / 24.6 / 20.6 / 22.8 / 26.5 us, 64: 67.3 / 47.9 / 37.9 / 43.9 / 62.6,
// 128: 68.4 / 54.8 / 51.9 / 59.4 / 80.5, 192: 78.0 / 65.9 / 69.2 / 79.2 /
// 102.7, 256: 80.8 / 79.4 / 78.2 / 92.2 / 120.9; n = 28672, K = 3: M = 64:
// 69.4 / 52.8 / 50.1 / 58.5 / 77.5, 128: 81.6 / 77.4 / 77.1 / 90.8 / 118.6;
// k = 14336, n = 4096, K = 3: M = 192: 230.9 / 128.8 / 84.9 / 68.7 / 68.0.
constexpr long long kFatHandoffWgs = 1024;
constexpr int kFatHandoffMinSteps = 16;

bool fat_handoff_on() { return env_int("EXL3_FAT_HANDOFF", 1) != 0; }

// EXL3_FAT_WIDE: 0 never wide tiles, 2 wide tiles whenever the shape allows
// them (M > kFatNarrowMaxRows, n a multiple of 256; tests of the wide
// kernel), otherwise the measured rule.
int fat_wide_mode() { return env_int("EXL3_FAT_WIDE", 1); }
bool fat_wide_allowed() { return fat_wide_mode() != 0; }

// Compute units of the current device (one wide-tile workgroup each), cached
// per device.
int fat_cus() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] <= 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
        cached[dev] = cus;
    }
    return cached[dev];
}

// Tiles of a one-split wide-tile launch that run as two k-halves (the tail
// split): the tiles of a last round that would fill at most half the CUs
// (or all tiles, when there are at most half as many as CUs).  Graph-timed,
// split vs whole (k = 4096, K = 3): gate/up n = 14336, M = 160 / 256 / 2048 /
// 2560: 96.7 / 99.9 / 546.9 / 678.0 vs 130.4 / 133.1 / 551.9 / 696.6 us;
// exl3_gemm n = 14336, M = 300 / 512: 91.8 / 95.4 vs 126.7 / 130.0, n = 28672,
// M = 768 / 2048: 221.7 / 522.2 vs 257.8 / 534.1.  Env EXL3_FAT_TAIL=0 turns
// it off.
int fat_tail_tiles(int tiles, int ksteps) {
    if (ksteps % 4 != 0 || env_int("EXL3_FAT_TAIL", 1) == 0) return 0;
    const int c = fat_cus(), r = tiles % c;
    return (r > 0 && 2 * r <= c) ? r : 0;
}
size_t fat_tail_bytes(int tail) { return (size_t)tail * FB_TAIL_FLOATS * sizeof(float); }

// Tail tiles of the wide kernel for an unsplit (m, k, n) call (gate/up mode:
// n per projection, one tile per 128-column block of each).
int wide_tail_tiles(int m, int k, int n, bool gu) {
    const int tiles = (gu ? n / 128 : n / FB_COLS) * ((m + FB_ROWS - 1) / FB_ROWS);
    return fat_tail_tiles(tiles, k / 64);
}

// f16out: a call with fp16 output (exl3_gemm), whose narrow k-splits use the
// partial-tile hand-off (fat_handoff) unless EXL3_FAT_HANDOFF=0.
FatPlan plan_fat(int M, int k, int n, bool f16out) {
    FatPlan pl;
    const int ksteps = k / 64;
    pl.splits = 1;
    if (fat_wide_allowed() && M > kFatNarrowMaxRows && n % FB_COLS == 0 &&
        (fat_wide_mode() == 2 || (long long)(n / FB_COLS) * ((M + FB_ROWS - 1) / FB_ROWS) >= kFatWideMinTiles)) {
        pl.mt = FAT_MT_WIDE;
        const long long base = (long long)(n / FB_COLS) * ((M + FB_ROWS - 1) / FB_ROWS);
        while (base * pl.splits < 96 && pl.splits < 16 && ksteps % (4 * pl.splits) == 0) pl.splits *= 2;
        return pl;
    }
    pl.mt = M > 16 ? 64 : 16;
    const int fmt = env_int("EXL3_FAT_MT", 0);  // tuning override: 16, 64 or 128 rows per tile
    if (fmt == 16 || fmt == 64 || fmt == 128) pl.mt = fmt;
    const long long base = (long long)(n / 128) * ((M + pl.mt - 1) / pl.mt);
    const bool ho = f16out && fat_handoff_on();
    const long long wgs = ho ? kFatHandoffWgs : kFatNarrowWgs;
    const int min_steps = ho ? kFatHandoffMinSteps : 0;
    const int forced = env_int("EXL3_FAT_SPLITS", 0);  // tuning override (power of two)
    while ((forced ? pl.splits < forced : base * pl.splits * 2 <= wgs && ksteps / (2 * pl.splits) >= min_steps) &&
           pl.splits < 16 && ksteps % (2 * pl.splits) == 0 && (ksteps / (2 * pl.splits)) % FAT_CH == 0)
        pl.splits *= 2;
    return pl;
}

int check_fat(const char* fn, const void* a, const void* trellis, const void* out, const void* svh, int M, int k,
              int n, int K, int cb) {
    EXL3_REQUIRE(M >= 0, "%s: M=%d", fn, M);
    EXL3_REQUIRE(k > 0 && n > 0 && k % 128 == 0 && n % 128 == 0, "%s: k=%d n=%d must be positive multiples of 128",
                 fn, k, n);
    EXL3_REQUIRE(K >= 1 && K <= 8, "%s: K=%d outside 1..8", fn, K);
    EXL3_REQUIRE(cb >= 0 && cb <= 2, "%s: codebook=%d outside 0..2", fn, cb);
    EXL3_REQUIRE(M == 0 || (a && trellis && out && svh), "%s: null pointer", fn);
    EXL3_REQUIRE(aligned(a, 16) && aligned(trellis, 16) && aligned(out, 8) && aligned(svh, 4),
                 "%s: misaligned pointer", fn);
    return EXL3_OK;
}

// Narrow 16-row tiles and wide tiles on mul1 weights read the raw entries
// (two VALU ops per two weights instead of four) and correct in the epilogue
// from the rotated rows' chunk sums.  Graph-timed, raw / decoded: config 3
// gate/up M = 16: 29.3 / 31.6 us, exl3_gemm k = 4096, n = 14336, M = 16:
// 22.7 / 23.2 us; on 64-row tiles the per-row sums cost more than the
// decode saves (gate/up M = 64: 55.8 / 53.7 us).  Wide tiles in gate/up mode
// sum a row's chunks in the epilogue, on the row's 8 lanes (config 3 M = 256
// / 2048: 89.4 / 478.9 -> 87.7 / 467.6 us); plain wide tiles stay decoded
// (exl3_gemm K = 3 mul1, n = 14336, M = 256 / 2048: 69.9 / 250.9 -> 70.3 /
// 250.3 us, each row's sums taken once per 128-column block).
// EXL3_FAT_RAW=0 turns it off (ablation).
bool fat_raw(int cb, int mt, bool gu) {
    return cb == 2 && (mt == 16 || (mt == FAT_MT_WIDE && gu)) && env_int("EXL3_FAT_RAW", 1) != 0;
}

// Narrow plans with k-splits and fp16 output hand partial tiles to the last
// split of each (column block, row tile) instead of adding fp32 atomically
// into a zero-filled buffer that a third launch converts.  EXL3_FAT_HANDOFF=0
// keeps the atomic path (ablation).
bool fat_handoff(const FatPlan& pl, int m, int n) {
    return pl.splits > 1 && pl.mt != FAT_MT_WIDE &&
           (size_t)(n / 128) * (size_t)((m + pl.mt - 1) / pl.mt) <= kWsMaxCounters && fat_handoff_on();
}

// Rows from which a 16-row tile's split hand-off goes to a finish launch
// (split_out; env EXL3_FAT_SPLIT_OUT=0: never).
constexpr int kSplitOutMinRows = 6;

// The second launch of a split-out hand-off: one wave per (row, column block).
int fat_split_finish(const FatParams& p, int splits, hipStream_t st, const char* what) {
    const unsigned wgs = (unsigned)(((long long)(p.n / 128) * p.M + 3) / 4);
    const bool raw = p.rowsum != nullptr;
    if (p.gu) {
        if (raw) fat_split_finish_kernel<true, true><<<wgs, 256, 0, st>>>(p, splits);
        else fat_split_finish_kernel<false, true><<<wgs, 256, 0, st>>>(p, splits);
    } else {
        if (raw) fat_split_finish_kernel<true, false><<<wgs, 256, 0, st>>>(p, splits);
        else fat_split_finish_kernel<false, false><<<wgs, 256, 0, st>>>(p, splits);
    }
    return launch_status(what);
}

// tail: tail-split tiles (unsplit wide launch with fp16 output; 0 = none),
// their hand-off tiles at tail_part and counts / flags at tail_sync.
// rowsum: chunk sums of a's rows, [M][k/128], for a raw-entry plan (else null).
// partials / counters: the split hand-off's partial tiles and counters
// (fat_handoff plans with fp16 output; else null).
int run_fat(const uint16_t* a, const int16_t* trellis, float* out32, __half* out16, const uint16_t* svh,
            const int64_t* token_idx, const uint16_t* route_w, int M, int k, int n, int K, int cb, bool zero_first,
            hipStream_t st, int tail = 0, char* tail_part = nullptr, int* tail_sync = nullptr,
            const float* rowsum = nullptr, float* partials = nullptr, int* counters = nullptr) {
    const FatPlan pl = plan_fat(M, k, n, out16 != nullptr);
    FatParams p{};
    if (partials && pl.splits > 1) {
        p.handoff = 1;
        p.partials = partials;
        p.counters = counters;
    }
    if (rowsum && fat_raw(cb, pl.mt, false)) p.rowsum = rowsum;
    if (tail > 0) {
        p.tiles_x = n / FB_COLS;
        p.tail_tiles = tail;
        p.tail_first = p.tiles_x * ((M + FB_ROWS - 1) / FB_ROWS) - tail;
        p.tail_part = reinterpret_cast<float*>(tail_part);
        p.tail_sync = tail_sync;
        p.max_polls = wait_polls();
        p.status = tail_sync + kWsStatusIndex;  // tail_sync is the workspace's counter region
    }
    p.a = reinterpret_cast<const __half*>(a);
    p.trellis = reinterpret_cast<const uint32_t*>(trellis);
    p.svh = reinterpret_cast<const __half*>(svh);
    p.out32 = out32;
    p.out16 = out16;
    p.token_idx = token_idx;
    p.route_w = reinterpret_cast<const __half*>(route_w);
    p.M = M;
    p.k = k;
    p.n = n;
    p.ksteps = k / 64 / pl.splits;
    const bool scatter = token_idx != nullptr;
    p.accumulate = (scatter || (pl.splits > 1 && !p.handoff)) ? 1 : 0;
    if (out16 && p.accumulate) {
        set_error("exl3 fat gemm: fp16 output needs a single k-split");
        return EXL3_ERR_UNSUPPORTED;
    }
    if (zero_first && p.accumulate && !scatter) {
        const size_t cnt = (size_t)M * n;
        fill_f32_kernel<<<(unsigned)((cnt + 255) / 256 < 4096 ? (cnt + 255) / 256 : 4096), 256, 0, st>>>(out32, cnt,
                                                                                                       0.f);
        const int rc = launch_status("exl3 fat gemm zero fill");
        if (rc) return rc;
    }
    // the split-out finish of the gate/up path, on the plain hand-off
    const bool split_out = p.handoff && pl.mt == 16 && M >= kSplitOutMinRows && pl.splits <= 4 &&
                           env_int("EXL3_FAT_SPLIT_OUT", 1) != 0;
    p.split_out = split_out ? 1 : 0;
    const int rc = fat_launch(K, cb, pl.mt, p, pl.splits, st);
    if (rc || !split_out) return rc;
    return fat_split_finish(p, pl.splits, st, "exl3 fat gemm finish launch");
}

}  // namespace

// Prefill path of exl3_gemm (m > gemm_gemv_rows(n)).  Scratch after the workspace's zeroed
// regions (shared with the GEMV kernels, which need them to stay zero); an
// unsplit GEMM stores fp16 straight to y.
// xr: the rotated rows (fp16 m*k), then their chunk sums (fp32 m*k/128).
size_t fat_xr_only_bytes(int m, int k) { return ((size_t)m * k * 2 + 255) & ~(size_t)255; }
size_t fat_xr_bytes(int m, int k) { return fat_xr_only_bytes(m, k) + (((size_t)m * (k / 128) * 4 + 255) & ~(size_t)255); }
// [counters][accumulators][xr][split partial tiles S*m*n fp32 (narrow
// hand-off) | out fp32 m*n (wide plan with k-splits) | tail-split hand-off
// tiles (unsplit wide launch)].
size_t fat_gemm_scratch_bytes(int m, int k, int n) {
    const FatPlan pl = plan_fat(m, k, n, true);
    const bool split = pl.splits > 1;
    const size_t tail = (!split && pl.mt == FAT_MT_WIDE) ? fat_tail_bytes(wide_tail_tiles(m, k, n, false)) : 0;
    const size_t out = fat_handoff(pl, m, n) ? (size_t)pl.splits * m * n * 4 : (size_t)m * n * 4;
    return kWsScratchOffset + fat_xr_bytes(m, k) + (split ? out : tail);
}

int fat_gemm_rows(const uint16_t* x, const int16_t* trellis, const uint16_t* suh, const uint16_t* svh, uint16_t* y,
                  int m, int k, int n, int K, int cb, void* ws, size_t ws_bytes, hipStream_t st) {
    const size_t need = fat_gemm_scratch_bytes(m, k, n);
    EXL3_REQUIRE_CODE(ws && ws_bytes >= need, EXL3_ERR_WORKSPACE,
                      "exl3_gemm: %zu workspace bytes needed for m=%d, %zu given", need, m,
                      ws ? ws_bytes : (size_t)0);
    EXL3_REQUIRE(aligned(x, 4) && aligned(y, 4) && aligned(suh, 4), "exl3_gemm: misaligned pointer");
    __half* xr = reinterpret_cast<__half*>(reinterpret_cast<char*>(ws) + kWsScratchOffset);
    float* o32 = reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + kWsScratchOffset + fat_xr_bytes(m, k));
    const FatPlan pl = plan_fat(m, k, n, true);
    float* rs = fat_raw(cb, pl.mt, false)
                    ? reinterpret_cast<float*>(reinterpret_cast<char*>(xr) + fat_xr_only_bytes(m, k))
                    : nullptr;
    const long long chunks = (long long)m * (k / 128);
    rotate_rows_kernel<<<(unsigned)((chunks + 3) / 4), 256, 0, st>>>(reinterpret_cast<const __half*>(x),
                                                                      reinterpret_cast<const __half*>(suh), xr, chunks,
                                                                      k, rs);
    int rc = launch_status("exl3_gemm rotate launch");
    if (rc) return rc;
    if (pl.splits == 1) {
        const int tail = pl.mt == FAT_MT_WIDE ? wide_tail_tiles(m, k, n, false) : 0;
        return run_fat(reinterpret_cast<const uint16_t*>(xr), trellis, nullptr, reinterpret_cast<__half*>(y), svh,
                       nullptr, nullptr, m, k, n, K, cb, false, st, tail, reinterpret_cast<char*>(o32),
                       reinterpret_cast<int*>(ws), rs);
    }
    if (fat_handoff(pl, m, n))
        return run_fat(reinterpret_cast<const uint16_t*>(xr), trellis, nullptr, reinterpret_cast<__half*>(y), svh,
                       nullptr, nullptr, m, k, n, K, cb, false, st, 0, nullptr, nullptr, rs, o32,
                       reinterpret_cast<int*>(ws));
    rc = run_fat(reinterpret_cast<const uint16_t*>(xr), trellis, o32, nullptr, svh, nullptr, nullptr, m, k, n, K, cb,
                 true, st, 0, nullptr, nullptr, rs);
    if (rc) return rc;
    const size_t n2 = (size_t)m * n / 2;
    f32_to_f16_kernel<<<(unsigned)((n2 + 255) / 256 < 8192 ? (n2 + 255) / 256 : 8192), 256, 0, st>>>(
        o32, reinterpret_cast<__half*>(y), n2);
    return launch_status("exl3_gemm convert launch");
}

// Gate/up SwiGLU on the MFMA kernels: the input is rotated once with the
// shared suh into the scratch, then
//   * up to kGateUpNarrowMaxRows rows: the narrow kernel in gate/up mode (16- or
//     64-row tiles; partial tiles and one counter per (column block, row tile)
//     in the scratch);
//   * above: the wide-tile kernel in gate/up mode (one split, tail split).
// k-splits of the narrow kernel: the most that keep the grid within 1.25 rounds
// of resident workgroups (CUs x waves per SIMD: 6 for 16-row tiles, set by
// their ~75 VGPRs, 4 for 64-row tiles, set by their LDS) and at least 16 steps
// per split (shorter splits spend more on the hand-off and epilogue than the
// extra workgroups win).  Config 3 (n = 14336 per projection, k = 4096),
// graph-timed, narrow splits 1 / 2 / 4 / 8: M = 16: 41.1 / 31.1 / 29.7 / 31.8
// us, 32: 57.0 / 42.0 / 39.7 / 43.2, 64: 80.1 / 57.1 / 56.6 / 64.4, 96: 80.6 /
// 68.5 / 74.1 / 88.6, 128: 89.0 / 79.2 / 81.0 / 96.8, 160: 93.7 / 106.0 / 98.7 /
// 118.0, 192: 106.8 / 110.9 / 109.8 / 132.8; wide tiles M = 160 / 192 / 256:
// 98.2 / 96.8 / 97.7.
constexpr int kGateUpNarrowMaxRows = 160;
constexpr int kGateUpMinSplitSteps = 16;

// Scratch: [counters][accumulators][xr fp16 m*k][partials, narrow only].
struct GateUpFatPlan {
    int mt, splits;
};

GateUpFatPlan plan_gate_up_fat(int m, int k, int n) {
    if (m > kGateUpNarrowMaxRows && fat_wide_allowed()) return GateUpFatPlan{FAT_MT_WIDE, 1};
    GateUpFatPlan pl{m <= 16 ? 16 : 64, 1};
    const int ksteps = k / 64;
    const long long base = 2LL * (n / 128) * ((m + pl.mt - 1) / pl.mt);
    const long long resident = (long long)fat_cus() * (pl.mt == 16 ? 6 : 4);
    const int min_steps = kGateUpMinSplitSteps;
    const int forced = env_int("EXL3_FAT_SPLITS", 0);  // tuning override (power of two)
    while ((forced ? pl.splits < forced
                   : base * pl.splits * 8 <= resident * 5 && ksteps / (2 * pl.splits) >= min_steps) &&
           pl.splits < 16 && ksteps % (2 * pl.splits) == 0 && (ksteps / (2 * pl.splits)) % FAT_CH == 0)
        pl.splits *= 2;
    return pl;
}

size_t fat_gate_up_scratch_bytes(int m, int k, int n) {
    const GateUpFatPlan pl = plan_gate_up_fat(m, k, n);
    size_t b = kWsScratchOffset + fat_xr_bytes(m, k);
    if (pl.mt != FAT_MT_WIDE) b += (size_t)2 * (n / 128) * pl.splits * (size_t)m * 128 * sizeof(float);
    else b += fat_tail_bytes(wide_tail_tiles(m, k, n, true));
    return b;
}

int fat_gate_up_rows(const uint16_t* x, const uint16_t* suh, const int16_t* gate_trellis, const uint16_t* gate_svh,
                     const int16_t* up_trellis, const uint16_t* up_svh, uint16_t* out, int m, int k, int n, int K,
                     int cb, float limit, void* ws, size_t ws_bytes, hipStream_t st) {
    const GateUpFatPlan pl = plan_gate_up_fat(m, k, n);
    const size_t need = fat_gate_up_scratch_bytes(m, k, n);
    EXL3_REQUIRE_CODE(ws && ws_bytes >= need, EXL3_ERR_WORKSPACE,
                      "exl3_gate_up_swiglu: %zu workspace bytes needed for m=%d, %zu given", need, m,
                      ws ? ws_bytes : (size_t)0);
    EXL3_REQUIRE(aligned(gate_trellis, 16) && aligned(up_trellis, 16) && aligned(gate_svh, 4) && aligned(up_svh, 4),
                 "exl3_gate_up_swiglu: misaligned pointer");
    const int mtiles = pl.mt == FAT_MT_WIDE ? 1 : (m + pl.mt - 1) / pl.mt;
    EXL3_REQUIRE_CODE((size_t)(n / 128) * mtiles <= kWsMaxCounters, EXL3_ERR_UNSUPPORTED,
                      "exl3_gate_up_swiglu: %d column blocks exceed the workspace counters", n / 128);
    char* w8 = reinterpret_cast<char*>(ws);
    __half* xr = reinterpret_cast<__half*>(w8 + kWsScratchOffset);
    float* rs = fat_raw(cb, pl.mt, true) ? reinterpret_cast<float*>(w8 + kWsScratchOffset + fat_xr_only_bytes(m, k)) : nullptr;
    const long long chunks = (long long)m * (k / 128);
    rotate_rows_kernel<<<(unsigned)((chunks + 3) / 4), 256, 0, st>>>(reinterpret_cast<const __half*>(x),
                                                                      reinterpret_cast<const __half*>(suh), xr, chunks,
                                                                      k, rs);
    int rc = launch_status("exl3_gate_up_swiglu rotate launch");
    if (rc) return rc;
    FatParams p{};
    p.rowsum = rs;
    p.a = xr;
    p.trellis = reinterpret_cast<const uint32_t*>(gate_trellis);
    p.svh = reinterpret_cast<const __half*>(gate_svh);
    p.trellis2 = reinterpret_cast<const uint32_t*>(up_trellis);
    p.svh2 = reinterpret_cast<const __half*>(up_svh);
    p.out16 = reinterpret_cast<__half*>(out);
    p.M = m;
    p.k = k;
    p.n = n;
    p.ksteps = k / 64 / pl.splits;
    p.gu = 1;
    p.limit = limit;
    p.counters = reinterpret_cast<int*>(w8);
    p.partials = reinterpret_cast<float*>(w8 + kWsScratchOffset + fat_xr_bytes(m, k));
    if (pl.mt == FAT_MT_WIDE) {
        const int tail = wide_tail_tiles(m, k, n, true);
        if (tail > 0) {
            p.tiles_x = n / 128;
            p.tail_tiles = tail;
            p.tail_first = p.tiles_x * ((m + FB_ROWS - 1) / FB_ROWS) - tail;
            p.tail_part = p.partials;
            p.tail_sync = p.counters;
            p.max_polls = wait_polls();
            p.status = p.counters + kWsStatusIndex;
        }
    }
    // One 16-row tile of 6 to 16 rows with up to 4 k-splits: the splits store
    // their partial tiles and exit, and fat_split_finish_kernel finishes every
    // (row, column block) in a launch of its own (env EXL3_FAT_SPLIT_OUT=0:
    // the in-kernel hand-off; same bits).  Config 3, graph-timed, in-kernel
    // hand-off -> finish launch: M = 4 / 6 / 8 / 10 / 12 / 14 / 16: 22.90 /
    // 24.48 / 24.95 / 26.1 / 26.21 / 27.1 / 27.22 -> 23.25 / 24.20 / 24.75 /
    // 25.07 / 25.45 / 25.8 / 26.1 us (with four rows the last arrival's chain
    // is short and the extra boundary does not pay).
    const bool split_out = pl.mt == 16 && m >= kSplitOutMinRows && pl.splits <= 4 &&
                           env_int("EXL3_FAT_SPLIT_OUT", 1) != 0;
    p.split_out = split_out ? 1 : 0;
    rc = fat_launch(K, cb, pl.mt, p, pl.splits, st);
    if (rc || !split_out) return rc;
    return fat_split_finish(p, pl.splits, st, "exl3_gate_up_swiglu finish launch");
}

}  // namespace exl3

using namespace exl3;

extern "C" int exl3_fat_gemm(const uint16_t* a, const int16_t* trellis, float* out, const uint16_t* svh, int M, int k,
                             int n, int K, int codebook, void* stream) {
    clear_error();
    int rc = check_fat("exl3_fat_gemm", a, trellis, out, svh, M, k, n, K, codebook);
    if (rc || M == 0) return rc;
    return run_fat(a, trellis, out, nullptr, svh, nullptr, nullptr, M, k, n, K, codebook, true, as_stream(stream));
}

extern "C" int exl3_fat_gemm_scatter(const uint16_t* a, const int16_t* trellis, float* out, const uint16_t* svh,
                                     const int64_t* token_idx, const uint16_t* route_weight, int M, int k, int n,
                                     int K, int codebook, void* stream) {
    clear_error();
    int rc = check_fat("exl3_fat_gemm_scatter", a, trellis, out, svh, M, k, n, K, codebook);
    if (rc || M == 0) return rc;
    EXL3_REQUIRE(token_idx && route_weight, "exl3_fat_gemm_scatter: null routing pointer");
    return run_fat(a, trellis, out, nullptr, svh, token_idx, route_weight, M, k, n, K, codebook, false,
                   as_stream(stream));
}

extern "C" size_t exl3_gemm_workspace_size(int m, int k, int n, int K) {
    if (m < 1 || k < 128 || n < 128) return 0;
    if (m <= gemm_gemv_rows(n)) return exl3_gemv_workspace_size(m, k, n, K, 1);
    return fat_gemm_scratch_bytes(m, k, n);
}
