"""Headline benchmark of the MI355X EXL3 path (one JSON line on stdout).

Headline metric: EXL3 GEMV packed-weight GB/s (% of HBM peak) at bs=1;
batched-MoE layer tokens/s.

A "step" is one exl3_gemv call of the headline shape (k=4096, n=14336, K=4,
MCG codebook, m=1) on seeded random trellis tiles and +-1 sign vectors.  The
calls cycle through 12 distinct weight copies (352 MB, more than the 256 MB
Infinity Cache) so every step streams its weight from HBM.  The K timed steps
are one HIP graph of K launches (no host overhead between kernels), bracketed
by HIP events on the launch stream, after W eager warmup launches and 0.2 s of
untimed replays of the same graph (steady clocks).  `value` = packed weight bytes per call /
time per call.  Extra fields: the m = 2/4/8 sweep and the CPU baseline (the
reference's CPU GEMV path restated in oracle/: truncating dequant + fp32
GEMM, single thread) timed on the host.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "sglang-exl3_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, published
K_DIM, N_DIM, BITS = 4096, 14336, 4
NCOPY = 12
WARM_S = 0.2  # untimed warm replay time before each timed graph replay


def make_weight(k, n, K, seed):
    rng = np.random.default_rng(seed)
    trellis = rng.integers(-32768, 32768, size=(k // 16, n // 16, 16 * K), dtype=np.int64).astype(np.int16)
    suh = np.where(rng.random(k) < 0.5, -1.0, 1.0).astype(np.float16)
    svh = np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float16)
    return trellis, suh, svh


def _warm_replays(torch, graph):
    """Untimed replays of `graph` for WARM_S seconds: the GPU's clocks settle
    under a load only after a few hundred milliseconds (a timed replay right
    after one warm replay read ~10 % slower than later ones)."""
    t_end = time.perf_counter() + WARM_S
    while True:
        graph.replay()
        torch.cuda.synchronize()
        if time.perf_counter() >= t_end:
            break


def gemv_timing(torch, L, weights, m, steps, warmup):
    """Median-free exact timing of `steps` graph-launched GEMVs; returns seconds per call."""
    k, n, K = K_DIM, N_DIM, BITS
    rng = np.random.default_rng(100 + m)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float16)).cuda()
    y = torch.empty((m, n), dtype=torch.float16, device="cuda")
    need = int(L.exl3_gemv_workspace_size(m, k, n, K, 1))
    ws = torch.zeros(max(need, 256), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    sp = int(stream.cuda_stream)

    def launch(c):
        tr, su, sv = weights[c % NCOPY]
        rc = L.exl3_gemv(x.data_ptr(), tr.data_ptr(), su.data_ptr(), sv.data_ptr(), y.data_ptr(), m, k, n, K, 1,
                         ws.data_ptr(), ws.numel(), sp)
        if rc:
            raise RuntimeError(L.exl3_last_error().decode())

    with torch.cuda.stream(stream):
        for c in range(max(warmup, 1)):
            launch(c)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            for c in range(steps):
                launch(c)
    torch.cuda.synchronize()
    _warm_replays(torch, graph)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        e0.record(stream)
        graph.replay()
        e1.record(stream)
    e1.synchronize()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e-3 / steps


# ------------------------------------------------------------- MoE layer (config 4)

MOE_E, MOE_TOPK, MOE_H, MOE_I, MOE_K = 128, 8, 2048, 768, 3
MOE_LAYERS = 2  # 2 x 226 MB of expert weights > the 256 MB Infinity Cache


def moe_routing(B, seed):
    """Config-4 router: logits N(0,1) + log p_e, p_e ~ rank^-1.1 over a seeded
    permutation of the experts; softmax, top-8, weights renormalised."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(MOE_E)
    p = (np.arange(1, MOE_E + 1, dtype=np.float64) ** -1.1)[np.argsort(perm)]
    p /= p.sum()
    logits = rng.standard_normal((B, MOE_E)) + np.log(p)[None, :]
    prob = np.exp(logits - logits.max(axis=1, keepdims=True))
    prob /= prob.sum(axis=1, keepdims=True)
    ids = np.argsort(-prob, axis=1)[:, :MOE_TOPK].astype(np.int32)
    w = np.take_along_axis(prob, ids, axis=1)
    w = (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
    return ids, w


class MoeWeights:
    """One layer's experts in three stacked device tensors per projection
    (trellis [E][k/16][n/16][16K], suh [E][k], svh [E][n]) plus the int64
    pointer tables the kernels read."""

    def __init__(self, torch, seed):
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        self.t = {}
        tabs = []
        for proj, k, n in (("gate", MOE_H, MOE_I), ("up", MOE_H, MOE_I), ("down", MOE_I, MOE_H)):
            tr = torch.randint(-32768, 32768, (MOE_E, k // 16, n // 16, 16 * MOE_K), dtype=torch.int16,
                               device="cuda", generator=g)
            su = (torch.randint(0, 2, (MOE_E, k), device="cuda", generator=g) * 2 - 1).half()
            # output scale 4/sqrt(k) folded into svh (as checkpoints do) keeps activations O(1)
            sv = ((torch.randint(0, 2, (MOE_E, n), device="cuda", generator=g) * 2 - 1) * (4.0 / k ** 0.5)).half()
            self.t[proj] = (tr, su, sv)
            for a in (tr, su, sv):
                step = a[0].numel() * a.element_size()
                tabs.append(torch.arange(MOE_E, dtype=torch.int64, device="cuda") * step + a.data_ptr())
        self.tables = tabs


def moe_loop(torch, x, ids_long, w, mw):
    """Per-expert loop over the same GEMV kernels, shaped like the reference's
    routed loop (src/sglang_exl3/exl3.py:520-576): unique experts on the host,
    gather, gate/up/down linears, SwiGLU, weighted index_add."""
    T = x.shape[0]
    out = torch.zeros((T, MOE_H), dtype=torch.float32, device=x.device)
    for e in torch.unique(ids_long).tolist():
        tok, slot = (ids_long == e).nonzero(as_tuple=True)
        h = x.index_select(0, tok)
        gt, gs, gv = (a[e] for a in mw.t["gate"])
        ut, us, uv = (a[e] for a in mw.t["up"])
        dt, ds, dv = (a[e] for a in mw.t["down"])
        gg = torch.ops.sglang_exl3.exl3_gemm(h, gt, gs, gv, MOE_K, True).float()
        uu = torch.ops.sglang_exl3.exl3_gemm(h, ut, us, uv, MOE_K, True).float()
        act = (torch.nn.functional.silu(gg) * uu).half()
        d = torch.ops.sglang_exl3.exl3_gemm(act, dt, ds, dv, MOE_K, True).float()
        out.index_add_(0, tok, d * w[tok, slot].unsqueeze(-1))
    return out


def moe_bench(torch, steps):
    from sglang_exl3 import ops

    ops.register_custom_ops()
    layers = [MoeWeights(torch, 1000 + i) for i in range(MOE_LAYERS)]
    torch.cuda.synchronize()
    res = {}
    for B in (1, 16, 64):
        ids_np, w_np = moe_routing(B, seed=B)
        U = len(np.unique(ids_np))
        x = torch.from_numpy(np.random.default_rng(B + 5).standard_normal((B, MOE_H)).astype(np.float16)).cuda()
        ids = torch.from_numpy(ids_np).cuda()
        w = torch.from_numpy(w_np).cuda()

        def layer(c):
            return torch.ops.sglang_exl3.exl3_moe_layer(x, ids, w, *layers[c % MOE_LAYERS].tables, MOE_K, MOE_K,
                                                        MOE_K, True, MOE_I, 0.0)

        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            for c in range(8):
                layer(c)
        torch.cuda.synchronize()
        # eager: back-to-back calls, host launch cost included
        n_eager = max(20, steps // 8)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            e0.record(stream)
            for c in range(n_eager):
                layer(c)
            e1.record(stream)
        e1.synchronize()
        t_eager = e0.elapsed_time(e1) * 1e-3 / n_eager
        # graph of `n` layer calls alternating the two layers
        n = max(24, steps // 4)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            with torch.cuda.graph(graph, stream=stream):
                for c in range(n):
                    layer(c)
        torch.cuda.synchronize()
        _warm_replays(torch, graph)
        with torch.cuda.stream(stream):
            e0.record(stream)
            graph.replay()
            e1.record(stream)
        e1.synchronize()
        t_graph = e0.elapsed_time(e1) * 1e-3 / n
        # per-expert loop of the same kernels
        ids_long = ids.long()
        for c in range(2):
            moe_loop(torch, x, ids_long, w, layers[c % MOE_LAYERS])
        torch.cuda.synchronize()
        n_loop = 6
        t0 = time.perf_counter()
        for c in range(n_loop):
            moe_loop(torch, x, ids_long, w, layers[c % MOE_LAYERS])
        torch.cuda.synchronize()
        t_loop = (time.perf_counter() - t0) / n_loop
        nbytes = U * (3 * MOE_H * MOE_I * MOE_K // 8)
        res[f"B{B}"] = {
            "unique_experts": U,
            "us_per_layer_graph": round(t_graph * 1e6, 2),
            "us_per_layer_eager": round(t_eager * 1e6, 2),
            "tokens_per_s": round(B / t_graph, 1),
            "GBps": round(nbytes / t_graph / 1e9, 1),
            "pct_hbm_peak": round(100 * nbytes / t_graph / 1e9 / HBM_PEAK_GBS, 2),
            "per_expert_loop_us": round(t_loop * 1e6, 1),
            "speedup_vs_loop_eager": round(t_loop / t_eager, 2),
        }
    return res


# -------------------------------------------------------- fat gate+up (config 3)

FAT_K, FAT_N, FAT_BITS, FAT_COPIES = 4096, 2 * 14336, 3, 8  # 8 x 44 MB > the Infinity Cache


def fat_bench(torch, L):
    """exl3_fat_gemm over the concatenated gate|up weight (mul1, K=3): rotated
    fp16 input, fp32 output; M=16 (HBM-bound) and M=2048 (MFMA-bound)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(31)
    trs = [torch.randint(-32768, 32768, (FAT_K // 16, FAT_N // 16, 16 * FAT_BITS), dtype=torch.int16, device="cuda",
                         generator=g) for _ in range(FAT_COPIES)]
    svh = ((torch.randint(0, 2, (FAT_N,), device="cuda", generator=g) * 2 - 1) * (4.0 / FAT_K ** 0.5)).half()
    res = {}
    for M, reps in ((16, 96), (2048, 16)):
        a = torch.randn(M, FAT_K, dtype=torch.float16, device="cuda", generator=g)
        out = torch.empty(M, FAT_N, dtype=torch.float32, device="cuda")
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())

        def launch(c):
            rc = L.exl3_fat_gemm(a.data_ptr(), trs[c % FAT_COPIES].data_ptr(), out.data_ptr(), svh.data_ptr(), M,
                                 FAT_K, FAT_N, FAT_BITS, 2, stream.cuda_stream)
            if rc:
                raise RuntimeError(L.exl3_last_error().decode())

        t = _graph_time(torch, stream, launch, reps)
        nbytes = FAT_K * FAT_N * FAT_BITS // 8
        flops = 2.0 * M * FAT_K * FAT_N
        res[f"M{M}"] = {"us_per_call": round(t * 1e6, 2), "TFLOPs": round(flops / t / 1e12, 1),
                        "pct_mfma_fp16_peak": round(100 * flops / t / 2.5e15, 2),
                        "GBps_packed": round(nbytes / t / 1e9, 1), "pct_hbm_peak": round(100 * nbytes / t / 8e12, 2),
                        "tokens_per_s": round(M / t, 1)}
    return res


def _graph_time(torch, stream, launch, reps):
    with torch.cuda.stream(stream):
        for c in range(3):
            launch(c)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            for c in range(reps):
                launch(c)
    torch.cuda.synchronize()
    _warm_replays(torch, graph)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        e0.record(stream)
        graph.replay()
        e1.record(stream)
    e1.synchronize()
    return e0.elapsed_time(e1) * 1e-3 / reps


# ---------------------------------------------------------- large MoE (config 5)

BIG_E, BIG_TOPK, BIG_H, BIG_I, BIG_M = 288, 8, 4096, 1536, 4
BIG_ROUTINGS = 8  # rotating uniform routings: the experts touched change every call


def big_moe_bench(torch):
    """288 routed experts (uniform top-8) + 1 shared expert (always taken, weight
    1) as one layer call, M=4 tokens; K in 2..5 with MCG (K=2, 4) and mul1
    (K=3, 5)."""
    res = {}
    rng = np.random.default_rng(55)
    E = BIG_E + 1  # the shared expert is expert BIG_E
    routings = []
    for r in range(BIG_ROUTINGS):
        ids = np.stack([rng.choice(BIG_E, BIG_TOPK, replace=False) for _ in range(BIG_M)])
        ids = np.concatenate([ids, np.full((BIG_M, 1), BIG_E)], axis=1).astype(np.int32)
        w = rng.random((BIG_M, BIG_TOPK)).astype(np.float32)
        w = np.concatenate([w / w.sum(1, keepdims=True), np.ones((BIG_M, 1), np.float32)], axis=1)
        routings.append((torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda(), len(np.unique(ids))))
    x = torch.randn(BIG_M, BIG_H, dtype=torch.float16, device="cuda")
    for K, mcg in ((2, True), (3, False), (4, True), (5, False)):
        g = torch.Generator(device="cuda")
        g.manual_seed(100 + K)
        tabs = []
        keep = []
        for k, n in ((BIG_H, BIG_I), (BIG_H, BIG_I), (BIG_I, BIG_H)):
            tr = torch.randint(-32768, 32768, (E, k // 16, n // 16, 16 * K), dtype=torch.int16, device="cuda",
                               generator=g)
            su = (torch.randint(0, 2, (E, k), device="cuda", generator=g) * 2 - 1).half()
            sv = ((torch.randint(0, 2, (E, n), device="cuda", generator=g) * 2 - 1) * (4.0 / k ** 0.5)).half()
            for a in (tr, su, sv):
                keep.append(a)
                tabs.append(torch.arange(E, dtype=torch.int64, device="cuda") * (a[0].numel() * a.element_size())
                            + a.data_ptr())
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())

        def launch(c):
            ids, w, _ = routings[c % BIG_ROUTINGS]
            torch.ops.sglang_exl3.exl3_moe_layer(x, ids, w, *tabs, K, K, K, mcg, BIG_I, 0.0)

        t = _graph_time(torch, stream, launch, 48)
        U = float(np.mean([u for _, _, u in routings]))
        nbytes = U * 3 * BIG_H * BIG_I * K / 8
        res[f"K{K}_{'mcg' if mcg else 'mul1'}"] = {
            "us_per_layer": round(t * 1e6, 2), "tokens_per_s": round(BIG_M / t, 1), "unique_experts": round(U, 2),
            "GBps": round(nbytes / t / 1e9, 1), "pct_hbm_peak": round(100 * nbytes / t / 8e12, 2)}
        del keep, tabs
        torch.cuda.empty_cache()
    return res


def profile_pass(torch, L, weights, steps):
    """Eager (non-graph) launches for rocprofv3: `steps` m=1 GEMVs over the rotating
    copies, then `steps` device copies of exactly one packed weight's bytes (the
    calibration kernel whose FETCH_SIZE / WRITE_SIZE readings scale the counters)."""
    k, n, K = K_DIM, N_DIM, BITS
    x = torch.from_numpy(np.random.default_rng(101).standard_normal((1, k)).astype(np.float16)).cuda()
    y = torch.empty((1, n), dtype=torch.float16, device="cuda")
    ws = torch.zeros(max(int(L.exl3_gemv_workspace_size(1, k, n, K, 1)), 256), dtype=torch.uint8, device="cuda")
    sp = int(torch.cuda.current_stream().cuda_stream)
    for c in range(steps):
        tr, su, sv = weights[c % NCOPY]
        rc = L.exl3_gemv(x.data_ptr(), tr.data_ptr(), su.data_ptr(), sv.data_ptr(), y.data_ptr(), 1, k, n, K, 1,
                         ws.data_ptr(), ws.numel(), sp)
        if rc:
            raise RuntimeError(L.exl3_last_error().decode())
    torch.cuda.synchronize()
    nbytes = k * n * K // 8
    src = [torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(c) for c in range(NCOPY)]
    dst = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    for c in range(steps):
        dst.copy_(src[c % NCOPY])
    torch.cuda.synchronize()
    print(json.dumps({"profile_pass": True, "gemv_launches": steps, "copy_launches": steps, "copy_bytes": nbytes}))


def cpu_baseline():
    """The reference's CPU exl3_gemv path (oracle restatement, one thread) on the full
    config-2 weight, m=1; median of 3 runs."""
    import oracle

    tr, su, sv = make_weight(K_DIM, N_DIM, BITS, seed=999)
    x = np.random.default_rng(5).standard_normal((1, K_DIM)).astype(np.float16)
    W = np.empty((K_DIM, N_DIM), dtype=np.uint16)
    ts = []
    for _ in range(3):
        t = time.perf_counter()
        oracle.cpu_gemv(x, tr, su, sv, BITS, 1, W)
        ts.append(time.perf_counter() - t)
    t = sorted(ts)[1]
    return {
        "value": round(K_DIM * N_DIM * BITS / 8 / t / 1e9, 5),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": "full config-2 weight (4096x14336, K=4, MCG), m=1: truncating dequant + fp32 GEMV, "
                  f"median of 3 runs, {t:.2f} s per call",
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=480)
    ap.add_argument("--warmup", type=int, default=48)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-moe", action="store_true", help="skip the batched-MoE layer leg")
    ap.add_argument("--no-extra", action="store_true", help="skip the config-3 and config-5 legs")
    ap.add_argument("--profile-pass", action="store_true",
                    help="eager m=1 launches plus a copy-kernel calibration, for rocprofv3 counter runs")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this path runs on one GPU; --gpus {args.gpus} is not supported "
              "(multi-GPU sharding is design-only)", file=sys.stderr)
        sys.exit(2)

    import torch

    from sglang_exl3 import _lib, ops

    L = _lib.lib()
    ops.register_custom_ops()
    weights = []
    for c in range(NCOPY):
        weights.append([torch.from_numpy(a).cuda() for a in make_weight(K_DIM, N_DIM, BITS, seed=c)])
    torch.cuda.synchronize()

    if args.profile_pass:
        profile_pass(torch, L, weights, args.steps)
        return

    bytes_per_call = K_DIM * N_DIM * BITS // 8
    t1 = gemv_timing(torch, L, weights, 1, args.steps, args.warmup)
    gbs = bytes_per_call / t1 / 1e9
    sweep = {}
    for m in (2, 4, 8):
        tm = gemv_timing(torch, L, weights, m, max(48, args.steps // 4), args.warmup)
        sweep[f"m{m}"] = {"us_per_call": round(tm * 1e6, 3), "GBps": round(bytes_per_call / tm / 1e9, 1),
                          "tokens_per_s": round(m / tm, 1)}
    plan = (__import__("ctypes").c_int * 5)()
    L.exl3_gemv_plan(1, K_DIM, N_DIM, BITS, 1, plan)

    traffic = None
    tf = os.path.join(ROOT, "profiles", "gemv_cfg2_m1_traffic.txt")
    if os.path.exists(tf):
        for line in open(tf):
            if line.startswith("hbm_bytes_per_launch:"):
                traffic = int(float(line.split(":", 1)[1]))

    result = {
        "metric": "EXL3 GEMV packed-weight GB/s (% of HBM peak) bs=1; batched-MoE layer tokens/s",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t1 * 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded random trellis, +-1 signs, x ~ N(0,1)); 12 rotating weight copies",
        "config": {"workload": "config 2: exl3_gemv k=4096 n=14336 K=4 MCG m=1",
                   "k": K_DIM, "n": N_DIM, "K": BITS, "codebook": "mcg", "m": 1,
                   "plan": {"row_blocks": plan[0], "steps_per_wave": plan[1], "k_waves": plan[2],
                            "k_splits": plan[3], "lds_bytes": plan[4]}},
        "pct_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "tokens_per_s": round(1.0 / t1, 1),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic},
        "gemv_sweep": sweep,
    }
    if not args.no_extra:
        result["fat_gate_up"] = {"config": "config 3: exl3_fat_gemm k=4096 n=2x14336 K=3 mul1, 8 rotating copies",
                                 **fat_bench(torch, L)}
        result["large_moe"] = {"config": "config 5: 288 experts top-8 uniform + shared, h=4096 I=1536, M=4, "
                                         "8 rotating routings", **big_moe_bench(torch)}
    if not args.no_moe:
        result["moe_layer"] = {"config": "config 4: E=128 top-8 hidden 2048 inter 768 K=3 MCG, "
                                         f"{MOE_LAYERS} rotating layer copies",
                               **moe_bench(torch, args.steps)}
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result))


if __name__ == "__main__":
    main()
