"""Headline benchmark of the MI355X EXL3 path (one JSON line on stdout).

Headline metric: EXL3 GEMV packed-weight GB/s (% of HBM peak) at bs=1;
batched-MoE layer tokens/s.

A "step" is one exl3_gemv call of the headline shape (config 2: k=4096,
n=14336, K=4, MCG codebook, m=1) on seeded random trellis tiles and +-1 sign
vectors.  Calls walk an endless cyclic sequence over 12 distinct weight copies
(352 MB, more than the 256 MB Infinity Cache): call c uses copy c % 12, so
every call's weight was last touched 11 copies (323 MB) earlier, whatever
--steps is.  The K timed steps are one HIP graph of K launches (no host
overhead between kernels), the next graph of that sequence, bracketed by
synchronisations and HIP events on the launch stream, after W eager warmup
launches and 0.2 s of untimed replays of the sequence (steady clocks).
`value` = packed weight bytes per call / time per call.

Further legs (each graph-timed the same way, with rotating inputs that keep
every call's weights out of the Infinity Cache): the m = 2/4/8 GEMV sweep,
config 3 (fused gate+up with the SwiGLU, fp16 out, M=16 and M=2048), config 5
(288+1 experts, M=4, K=2..5), config 4 (128 experts top-8, B=1/16/64, against a
graph-captured per-expert loop of the same kernels and against the reference's
host-synced loop), and the CPU baseline: config 1 on the reference's CPU path
as restated in oracle/ (truncating dequant on one core, then the fp32 GEMV by
torch on 1 and on all host threads).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "sglang-exl3_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, published
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA, published
K_DIM, N_DIM, BITS = 4096, 14336, 4
NCOPY = 12
WARM_S = 0.2  # untimed warm replay time before each timed graph replay
ANTI_CACHE_BYTES = 300e6  # bytes touched between two uses of one weight copy (> 256 MB Infinity Cache)


def make_weight(k, n, K, seed):
    rng = np.random.default_rng(seed)
    trellis = rng.integers(-32768, 32768, size=(k // 16, n // 16, 16 * K), dtype=np.int64).astype(np.int16)
    suh = np.where(rng.random(k) < 0.5, -1.0, 1.0).astype(np.float16)
    svh = np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float16)
    return trellis, suh, svh


def _sign_f16(torch, n, g, scale=1.0):
    return ((torch.randint(0, 2, (n,), device="cuda", generator=g) * 2 - 1) * scale).half()


def _rand_trellis(torch, shape, g):
    return torch.randint(-32768, 32768, shape, dtype=torch.int16, device="cuda", generator=g)


# --------------------------------------------------------------- timing core

def seq_time(torch, stream, launch, n, period, warmup=3):
    """Seconds per call of `launch(c)` for an endless call sequence c = 0, 1, ...
    in which call c uses input set c % period.  The sequence is cut into HIP
    graphs of n calls (graph j holds calls j n .. j n + n - 1, G = period /
    gcd(n, period) graphs); replaying them in order continues the sequence, so
    every call's inputs were last used exactly `period` calls earlier whatever
    n is.  Eager warmup calls, then WARM_S seconds of replays (steady clocks),
    then the next graph is timed with HIP events on `stream`, synchronised on
    both sides."""
    G = period // math.gcd(n, period)
    with torch.cuda.stream(stream):
        for c in range(max(warmup, 1)):
            launch(c)
    torch.cuda.synchronize()
    graphs = []
    for j in range(G):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            with torch.cuda.graph(g, stream=stream):
                for i in range(n):
                    launch(j * n + i)
        graphs.append(g)
    torch.cuda.synchronize()
    t_end = time.perf_counter() + WARM_S
    with torch.cuda.stream(stream):
        while True:
            for g in graphs:
                g.replay()
            torch.cuda.synchronize()
            if time.perf_counter() >= t_end:
                break
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        graphs[0].replay()
        e1.record(stream)
    e1.synchronize()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e-3 / n


def _log(msg):
    """Progress line on stderr (stdout carries only the JSON result)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _stream(torch):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    return s


# ------------------------------------------------------------ GEMV (config 2)

def gemv_weights(torch):
    g = torch.Generator(device="cuda")
    g.manual_seed(2)
    return [(_rand_trellis(torch, (K_DIM // 16, N_DIM // 16, 16 * BITS), g), _sign_f16(torch, K_DIM, g),
             _sign_f16(torch, N_DIM, g)) for _ in range(NCOPY)]


def gemv_timing(torch, L, weights, m, steps, warmup):
    """Seconds per exl3_gemv call of [m, 4096] x [4096, 14336] over the rotating copies."""
    k, n, K = K_DIM, N_DIM, BITS
    rng = np.random.default_rng(100 + m)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float16)).cuda()
    y = torch.empty((m, n), dtype=torch.float16, device="cuda")
    need = int(L.exl3_gemv_workspace_size(m, k, n, K, 1))
    ws = torch.zeros(max(need, 256), dtype=torch.uint8, device="cuda")
    stream = _stream(torch)
    sp = int(stream.cuda_stream)

    def launch(c):
        tr, su, sv = weights[c % NCOPY]
        rc = L.exl3_gemv(x.data_ptr(), tr.data_ptr(), su.data_ptr(), sv.data_ptr(), y.data_ptr(), m, k, n, K, 1,
                         ws.data_ptr(), ws.numel(), sp)
        if rc:
            raise RuntimeError(L.exl3_last_error().decode())

    return seq_time(torch, stream, launch, steps, NCOPY, warmup)


# ---------------------------------------------------- fused gate+up (config 3)

GU_K, GU_N, GU_BITS = 4096, 14336, 3
GU_COPIES = 8  # 8 x 44 MB of gate+up packs: 7 copies (308 MB) between two uses of one


def gate_up_bench(torch):
    """exl3_gate_up_swiglu on config 3: x [M, 4096] -> fp16 silu(gate) * up [M, 14336], gate and up
    14336 wide each, K=3 mul1; M=16 (decode, HBM-bound) and M=2048 (prefill, MFMA-bound)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(31)
    shape = (GU_K // 16, GU_N // 16, 16 * GU_BITS)
    packs = [(_rand_trellis(torch, shape, g), _rand_trellis(torch, shape, g)) for _ in range(GU_COPIES)]
    suh = _sign_f16(torch, GU_K, g)
    svg = _sign_f16(torch, GU_N, g, 4.0 / GU_K ** 0.5)
    svu = _sign_f16(torch, GU_N, g, 4.0 / GU_K ** 0.5)
    res = {}
    nbytes = 2 * GU_K * GU_N * GU_BITS // 8
    for M, n in ((16, 48), (2048, 16)):
        x = torch.randn(M, GU_K, dtype=torch.float16, device="cuda", generator=g)
        stream = _stream(torch)

        def launch(c):
            tg, tu = packs[c % GU_COPIES]
            torch.ops.sglang_exl3.exl3_gate_up_swiglu(x, suh, tg, svg, tu, svu, GU_BITS, 2, 0.0)

        t = seq_time(torch, stream, launch, n, GU_COPIES)
        flops = 2.0 * M * GU_K * 2 * GU_N
        res[f"M{M}"] = {"us_per_call": round(t * 1e6, 2), "TFLOPs": round(flops / t / 1e12, 1),
                        "pct_mfma_fp16_peak": round(100 * flops / t / 1e12 / MFMA_F16_PEAK_TFLOPS, 2),
                        "GBps_packed": round(nbytes / t / 1e9, 1),
                        "pct_hbm_peak": round(100 * nbytes / t / 1e9 / HBM_PEAK_GBS, 2),
                        "tokens_per_s": round(M / t, 1)}
    return res


# ------------------------------------------------------------- MoE (config 4)

MOE_E, MOE_TOPK, MOE_H, MOE_I, MOE_K = 128, 8, 2048, 768, 3
MOE_EXPERT_BYTES = 3 * MOE_H * MOE_I * MOE_K // 8  # 1,769,472 B
MOE_LAYER_COPIES = 24  # 24 x 226 MB of expert weights
MOE_ROUTINGS = 8       # rotating routings per batch size


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
            tr = _rand_trellis(torch, (MOE_E, k // 16, n // 16, 16 * MOE_K), g)
            su = (torch.randint(0, 2, (MOE_E, k), device="cuda", generator=g) * 2 - 1).half()
            # output scale 4/sqrt(k) folded into svh (as checkpoints do) keeps activations O(1)
            sv = ((torch.randint(0, 2, (MOE_E, n), device="cuda", generator=g) * 2 - 1) * (4.0 / k ** 0.5)).half()
            self.t[proj] = (tr, su, sv)
            for a in (tr, su, sv):
                step = a[0].numel() * a.element_size()
                tabs.append(torch.arange(MOE_E, dtype=torch.int64, device="cuda") * step + a.data_ptr())
        self.tables = tabs


def loop_plan(torch, ids_np, w_np):
    """Per active expert: its token rows and routing weights as device tensors
    (what the reference's loop finds with torch.unique / nonzero on the host)."""
    plan = []
    for e in np.unique(ids_np):
        tok, slot = np.nonzero(ids_np == e)
        plan.append((int(e), torch.from_numpy(tok.astype(np.int64)).cuda(),
                     torch.from_numpy(w_np[tok, slot].astype(np.float32)).cuda()[:, None]))
    return plan


def moe_loop_static(torch, x, plan, mw):
    """Per-expert loop of the same GEMV kernels (gather, gate, up, SwiGLU, down,
    weighted index_add: the shape of src/sglang_exl3/exl3.py:520-576) with the
    routing resolved beforehand, so it can be captured in a graph."""
    out = torch.zeros((x.shape[0], MOE_H), dtype=torch.float32, device=x.device)
    for e, tok, wv in plan:
        h = x.index_select(0, tok)
        gg = torch.ops.sglang_exl3.exl3_gemm(h, *(a[e] for a in mw.t["gate"]), MOE_K, True).float()
        uu = torch.ops.sglang_exl3.exl3_gemm(h, *(a[e] for a in mw.t["up"]), MOE_K, True).float()
        act = (torch.nn.functional.silu(gg) * uu).half()
        d = torch.ops.sglang_exl3.exl3_gemm(act, *(a[e] for a in mw.t["down"]), MOE_K, True).float()
        out.index_add_(0, tok, d * wv)
    return out


def moe_loop_eager(torch, x, ids_long, w, mw):
    """The reference's routed loop as it runs: unique experts and their rows
    found on the host every call (host-synchronising), then the same kernels."""
    out = torch.zeros((x.shape[0], MOE_H), dtype=torch.float32, device=x.device)
    for e in torch.unique(ids_long).tolist():
        tok, slot = (ids_long == e).nonzero(as_tuple=True)
        h = x.index_select(0, tok)
        gg = torch.ops.sglang_exl3.exl3_gemm(h, *(a[e] for a in mw.t["gate"]), MOE_K, True).float()
        uu = torch.ops.sglang_exl3.exl3_gemm(h, *(a[e] for a in mw.t["up"]), MOE_K, True).float()
        act = (torch.nn.functional.silu(gg) * uu).half()
        d = torch.ops.sglang_exl3.exl3_gemm(act, *(a[e] for a in mw.t["down"]), MOE_K, True).float()
        out.index_add_(0, tok, d * w[tok, slot].unsqueeze(-1))
    return out


def moe_bench(torch):
    """Config 4 layer calls over rotating layer copies and routings: call c uses
    layer copy c % L and routing c % R, with L chosen so that more than 300 MB of
    other experts' weights are touched between two uses of one copy."""
    layers = [MoeWeights(torch, 1000 + i) for i in range(MOE_LAYER_COPIES)]
    torch.cuda.synchronize()
    res = {}
    for B in (1, 16, 64):
        routings = [moe_routing(B, seed=B * 1000 + r) for r in range(MOE_ROUTINGS)]
        us = [len(np.unique(ids)) for ids, _ in routings]
        U = float(np.mean(us))
        per_call = U * MOE_EXPERT_BYTES
        nl = min(MOE_LAYER_COPIES, int(math.ceil(ANTI_CACHE_BYTES / per_call)) + 1)
        period = nl * MOE_ROUTINGS // math.gcd(nl, MOE_ROUTINGS)
        x = torch.from_numpy(np.random.default_rng(B + 5).standard_normal((B, MOE_H)).astype(np.float16)).cuda()
        dev_r = [(torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()) for ids, w in routings]

        def layer(c):
            ids, w = dev_r[c % MOE_ROUTINGS]
            return torch.ops.sglang_exl3.exl3_moe_layer(x, ids, w, *layers[c % nl].tables, MOE_K, MOE_K, MOE_K,
                                                        True, MOE_I, 0.0)

        stream = _stream(torch)
        t_graph = seq_time(torch, stream, layer, 48, period)
        # eager: back-to-back calls through the same sequence, host launch cost included
        n_eager = 48
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            torch.cuda.synchronize()
            e0.record(stream)
            for c in range(n_eager):
                layer(c)
            e1.record(stream)
        e1.synchronize()
        t_eager = e0.elapsed_time(e1) * 1e-3 / n_eager
        # per-expert loop of the same kernels, routing resolved beforehand, graph-timed
        plans = [loop_plan(torch, ids, w) for ids, w in routings]

        def loop(c):
            return moe_loop_static(torch, x, plans[c % MOE_ROUTINGS], layers[c % nl])

        # every routing x layer shape once eagerly first: the per-stream workspace of exl3_gemm is sized
        # by the rows per expert, and it may not grow during capture
        t_loop_graph = seq_time(torch, stream, loop, 8, period, warmup=period)
        # the reference's host-synced loop, eager
        for c in range(2):
            ids, w = dev_r[c % MOE_ROUTINGS]
            moe_loop_eager(torch, x, ids.long(), w, layers[c % nl])
        torch.cuda.synchronize()
        n_loop = 6
        t0 = time.perf_counter()
        for c in range(n_loop):
            ids, w = dev_r[c % MOE_ROUTINGS]
            moe_loop_eager(torch, x, ids.long(), w, layers[c % nl])
        torch.cuda.synchronize()
        t_loop_eager = (time.perf_counter() - t0) / n_loop
        _log(f"config 4 B={B}: layer {t_graph * 1e6:.1f} us, loop {t_loop_graph * 1e6:.1f} us")
        res[f"B{B}"] = {
            "unique_experts_mean": round(U, 2),
            "layer_copies": nl,
            "bytes_between_reuse_MB": round((nl - 1) * per_call / 1e6, 1),
            "us_per_layer_graph": round(t_graph * 1e6, 2),
            "us_per_layer_eager": round(t_eager * 1e6, 2),
            "tokens_per_s": round(B / t_graph, 1),
            "GBps": round(per_call / t_graph / 1e9, 1),
            "pct_hbm_peak": round(100 * per_call / t_graph / 1e9 / HBM_PEAK_GBS, 2),
            "per_expert_loop_graph_us": round(t_loop_graph * 1e6, 1),
            "speedup_vs_loop_graph": round(t_loop_graph / t_graph, 2),
            "per_expert_loop_eager_us": round(t_loop_eager * 1e6, 1),
            "speedup_vs_loop_eager": round(t_loop_eager / t_eager, 2),
        }
    return res


# ---------------------------------------------------------- large MoE (config 5)

BIG_E, BIG_TOPK, BIG_H, BIG_I, BIG_M = 288, 8, 4096, 1536, 4
BIG_ROUTINGS = 8  # rotating uniform routings: the experts touched change every call


def big_moe_bench(torch):
    """288 routed experts (uniform top-8) + 1 shared expert (always taken, weight
    1) as one layer call, M=4 tokens; K in 2..5 with MCG (K=2, 4) and mul1
    (K=3, 5).  Each call touches ~32 experts (>= 450 MB at K=2), so the weights
    stream from HBM."""
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
            tr = _rand_trellis(torch, (E, k // 16, n // 16, 16 * K), g)
            su = (torch.randint(0, 2, (E, k), device="cuda", generator=g) * 2 - 1).half()
            sv = ((torch.randint(0, 2, (E, n), device="cuda", generator=g) * 2 - 1) * (4.0 / k ** 0.5)).half()
            for a in (tr, su, sv):
                keep.append(a)
                tabs.append(torch.arange(E, dtype=torch.int64, device="cuda") * (a[0].numel() * a.element_size())
                            + a.data_ptr())
        stream = _stream(torch)

        def launch(c):
            ids, w, _ = routings[c % BIG_ROUTINGS]
            torch.ops.sglang_exl3.exl3_moe_layer(x, ids, w, *tabs, K, K, K, mcg, BIG_I, 0.0)

        t = seq_time(torch, stream, launch, 48, BIG_ROUTINGS)
        U = float(np.mean([u for _, _, u in routings]))
        nbytes = U * 3 * BIG_H * BIG_I * K / 8
        res[f"K{K}_{'mcg' if mcg else 'mul1'}"] = {
            "us_per_layer": round(t * 1e6, 2), "tokens_per_s": round(BIG_M / t, 1), "unique_experts": round(U, 2),
            "GBps": round(nbytes / t / 1e9, 1), "pct_hbm_peak": round(100 * nbytes / t / 1e9 / HBM_PEAK_GBS, 2)}
        del keep, tabs
        torch.cuda.empty_cache()
    return res


# ------------------------------------------------------------ profile passes

def profile_pass(torch, L, kind, steps, moe_batch=16):
    """Eager launches for rocprofv3 counter runs, then `steps` device copies of a
    known byte count (the calibration kernel whose FETCH_SIZE / WRITE_SIZE
    readings scale the counters).
      gemv: `steps` m=1 config-2 GEMVs over the rotating copies (copy: one packed weight);
      moe:  `steps` config-4 layer calls at B = `moe_batch` (16 by default) over 8 layer copies
            (copy: 16 experts' packs);
      gate_up: `steps` config-3 exl3_gate_up_swiglu calls at M=16 over the 8 pack copies (copy: one
            gate+up pair's packed bytes);
      gate_up_prefill: the same at M=2048 (`steps` // 4 calls and copies)."""
    if kind == "gemv":
        weights = gemv_weights(torch)
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
        nbytes = k * n * K // 8
        ncopy = NCOPY
    elif kind in ("gate_up", "gate_up_prefill"):
        g = torch.Generator(device="cuda")
        g.manual_seed(31)
        shape = (GU_K // 16, GU_N // 16, 16 * GU_BITS)
        packs = [(_rand_trellis(torch, shape, g), _rand_trellis(torch, shape, g)) for _ in range(GU_COPIES)]
        suh = _sign_f16(torch, GU_K, g)
        svg = _sign_f16(torch, GU_N, g, 4.0 / GU_K ** 0.5)
        svu = _sign_f16(torch, GU_N, g, 4.0 / GU_K ** 0.5)
        M = 2048 if kind == "gate_up_prefill" else 16
        if M > 16:
            steps = max(1, steps // 4)
        x = torch.randn(M, GU_K, dtype=torch.float16, device="cuda", generator=g)
        for c in range(steps):
            tg, tu = packs[c % GU_COPIES]
            torch.ops.sglang_exl3.exl3_gate_up_swiglu(x, suh, tg, svg, tu, svu, GU_BITS, 2, 0.0)
        nbytes = 2 * GU_K * GU_N * GU_BITS // 8
        ncopy = GU_COPIES
    else:
        layers = [MoeWeights(torch, 1000 + i) for i in range(8)]
        B = moe_batch
        ids, w = moe_routing(B, seed=B * 1000)
        x = torch.from_numpy(np.random.default_rng(B + 5).standard_normal((B, MOE_H)).astype(np.float16)).cuda()
        idd, wd = torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()
        for c in range(steps):
            torch.ops.sglang_exl3.exl3_moe_layer(x, idd, wd, *layers[c % 8].tables, MOE_K, MOE_K, MOE_K, True, MOE_I,
                                                 0.0)
        nbytes = 16 * MOE_EXPERT_BYTES
        ncopy = 8
    torch.cuda.synchronize()
    src = [torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(c) for c in range(ncopy)]
    dst = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    for c in range(steps):
        dst.copy_(src[c % ncopy])
    torch.cuda.synchronize()
    print(json.dumps({"profile_pass": kind, "launches": steps, "copy_launches": steps, "copy_bytes": nbytes}))


# --------------------------------------------------------------- CPU baseline

def cpu_baseline(torch):
    """Config 1 on the reference's CPU path (src/sglang_exl3/ops.py -> csrc/bindings.cpp:117-147:
    dequant_cpu, then at::mm in fp32), restated: oracle.dequant (truncating decode, two fp32 FWHT
    passes; one core, as the reference) and torch.mm in fp32 on 1 and on all host threads.
    Median of 5 runs after one warm-up; `value` is packed-weight GB/s of the whole call at all threads."""
    import oracle

    k = n = 4096
    K = 4
    tr, su, sv = make_weight(k, n, K, seed=0)
    x = np.random.default_rng(0).standard_normal((1, k)).astype(np.float16)
    reps = 5
    nthreads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    saved = torch.get_num_threads()

    def med(f):
        f()
        ts = []
        for _ in range(reps):
            t = time.perf_counter()
            f()
            ts.append(time.perf_counter() - t)
        return sorted(ts)[reps // 2]

    W = oracle.dequant(tr, su, sv, K, 1, rtz=True)
    t_dq = med(lambda: oracle.dequant(tr, su, sv, K, 1, rtz=True))
    xt = torch.from_numpy(x.astype(np.float32))
    Wt = torch.from_numpy(W.view(np.float16).astype(np.float32))
    mm = {}
    for th in (1, nthreads):
        torch.set_num_threads(th)
        mm[th] = med(lambda: torch.mm(xt, Wt).half())
    torch.set_num_threads(saved)
    total = t_dq + mm[nthreads]
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    nbytes = k * n * K // 8
    return {
        "value": round(nbytes / total / 1e9, 5),
        "unit": "GB/s",
        "cores": nthreads,
        "kind": "port",
        "sample": f"config 1 (4096x4096, K=4, MCG, m=1), whole call, median of {reps} after one warm-up: "
                  f"dequant {t_dq:.3f} s on 1 core + fp32 GEMV {mm[nthreads] * 1e3:.2f} ms on {nthreads} threads",
        "dequant_s_1core": round(t_dq, 4),
        "gemv_fp32_ms_1thread": round(mm[1] * 1e3, 3),
        f"gemv_fp32_ms_{nthreads}threads": round(mm[nthreads] * 1e3, 3),
        "total_s": round(total, 4),
        "tokens_per_s": round(1.0 / total, 3),
        "cpu": cpu_model,
        "torch_threads_default": saved,
    }


# ----------------------------------------------------------------------- main

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=480)
    ap.add_argument("--warmup", type=int, default=48)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-moe", action="store_true", help="skip the batched-MoE layer leg")
    ap.add_argument("--no-extra", action="store_true", help="skip the config-3 and config-5 legs")
    ap.add_argument("--profile-pass", choices=("gemv", "moe", "gate_up", "gate_up_prefill"),
                    help="eager launches plus a copy-kernel calibration, for rocprofv3 counter runs")
    ap.add_argument("--moe-batch", type=int, default=16, choices=(1, 16, 64),
                    help="tokens per layer call of --profile-pass moe")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this path runs on one GPU; --gpus {args.gpus} is not supported "
              "(multi-GPU sharding is design-only)", file=sys.stderr)
        sys.exit(2)

    import torch

    from sglang_exl3 import _lib, ops

    L = _lib.lib()
    ops.register_custom_ops()
    if args.profile_pass:
        profile_pass(torch, L, args.profile_pass, args.steps, args.moe_batch)
        return

    weights = gemv_weights(torch)
    torch.cuda.synchronize()
    bytes_per_call = K_DIM * N_DIM * BITS // 8
    t1 = gemv_timing(torch, L, weights, 1, args.steps, args.warmup)
    gbs = bytes_per_call / t1 / 1e9
    _log(f"gemv m=1: {t1 * 1e6:.2f} us")
    sweep = {}
    for m in (2, 4, 8):
        tm = gemv_timing(torch, L, weights, m, max(48, args.steps // 4), args.warmup)
        sweep[f"m{m}"] = {"us_per_call": round(tm * 1e6, 3), "GBps": round(bytes_per_call / tm / 1e9, 1),
                          "pct_hbm_peak": round(100 * bytes_per_call / tm / 1e9 / HBM_PEAK_GBS, 2),
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
        "data": "synthetic (seeded random trellis, +-1 signs, x ~ N(0,1)); 12 weight copies in a cyclic "
                "sequence (323 MB between two uses of one copy)",
        "config": {"workload": "config 2: exl3_gemv k=4096 n=14336 K=4 MCG m=1",
                   "k": K_DIM, "n": N_DIM, "K": BITS, "codebook": "mcg", "m": 1, "weight_copies": NCOPY,
                   "plan": {"row_blocks": plan[0], "steps_per_wave": plan[1], "k_waves": plan[2],
                            "k_splits": plan[3], "lds_bytes": plan[4]}},
        "pct_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "tokens_per_s": round(1.0 / t1, 1),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": ("profiles/gemv_cfg2_m1_traffic.txt: rocprofv3 FETCH_SIZE + WRITE_SIZE of "
                                        "this kernel from a profiled run (bench.py --profile-pass gemv), not "
                                        "measured in this run") if traffic is not None else None},
        "gemv_sweep": sweep,
    }
    if not args.no_extra:
        _log("gemv sweep done")
        result["gate_up_swiglu"] = {"config": "config 3: exl3_gate_up_swiglu k=4096, gate and up 14336 each, "
                                              "K=3 mul1, fp16 SiLU(gate)*up out, 8 rotating copies",
                                    **gate_up_bench(torch)}
        _log("config 3 done")
        result["large_moe"] = {"config": "config 5: 288 experts top-8 uniform + shared, h=4096 I=1536, M=4, "
                                         "8 rotating routings", **big_moe_bench(torch)}
        _log("config 5 done")
    if not args.no_moe:
        result["moe_layer"] = {"config": "config 4: E=128 top-8 (Zipf 1.1 router) hidden 2048 inter 768 K=3 MCG; "
                                         "rotating layer copies x 8 routings, >300 MB between reuses",
                               **moe_bench(torch)}
        _log("config 4 done")
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(torch)
        _log("cpu baseline done")
    print(json.dumps(result))


if __name__ == "__main__":
    main()
