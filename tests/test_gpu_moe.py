"""GPU parity of the batched MoE layer (exl3_moe_layer) and the one-token fused
MoE (p2b_fused_moe) against the CPU oracle's routed loop.

The oracle (oracle.moe_ref) follows src/sglang_exl3/exl3.py:520-576: per expert,
gate/up linears of the fp16 tokens in fp32, silu(min(g, L)) * clamp(u, -L, L),
the activation cast to fp16, the down linear, out[t] += w * down.  The GPU path
rounds gate/up to fp16 as the batched reference path does (exl3.py:1018-1034);
both sit inside the bar: max-abs-err <= 2e-2 * rms(ref), cosine >= 0.9999.
"""

import numpy as np
import pytest
import torch

import oracle
from gpu_util import check_close, make_weight, make_x
from sglang_exl3 import _lib, ops

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _registered():
    ops.register_custom_ops()


class Experts:
    """E experts with seeded weights: numpy copies for the oracle, device tensors
    kept alive behind int64 pointer tables (the layout of exl3.py:590-607)."""

    def __init__(self, E, hidden, inter, Ks=(3, 3, 3), cb=1, seed=0):
        self.E, self.hidden, self.inter, self.Ks, self.cb = E, hidden, inter, Ks, cb
        self.np = []
        self.dev = []
        cols = {p: ([], [], []) for p in ("gate", "up", "down")}
        for e in range(E):
            spec = {}
            for j, (proj, k, n) in enumerate((("gate", hidden, inter), ("up", hidden, inter), ("down", inter, hidden))):
                K = Ks[j]
                tr, su, sv = make_weight(k, n, K, seed=seed * 100003 + 3 * e + j)
                # output scale folded into svh, as real checkpoints do, so that
                # activations stay O(1) and fp16 never overflows: W ~ 4/sqrt(k)
                sv = (sv.astype(np.float32) * (4.0 / np.sqrt(k))).astype(np.float16)
                spec[proj] = (tr, su, sv, K, cb)
                d = [torch.from_numpy(a).cuda() for a in (tr, su, sv)]
                self.dev.append(d)
                for c, t in zip(cols[proj], d):
                    c.append(t.data_ptr())
            self.np.append(spec)
        self.tables = []
        for proj in ("gate", "up", "down"):
            for c in cols[proj]:
                self.tables.append(torch.tensor(c, dtype=torch.int64, device="cuda"))

    def layer(self, x, ids, w, limit=0.0):
        KG, KU, KD = self.Ks
        return torch.ops.sglang_exl3.exl3_moe_layer(x, ids, w, *self.tables, KG, KU, KD, self.cb == 1, self.inter,
                                                    limit)

    def ref(self, x_np, ids_np, w_np, limit=float("inf")):
        return oracle.moe_ref(x_np, ids_np, w_np, self.np, limit)


def _routing(T, topk, E, seed, invalid=0):
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.choice(E, size=topk, replace=False) for _ in range(T)]).astype(np.int32)
    w = rng.random((T, topk)).astype(np.float32) + 0.05
    w /= w.sum(axis=1, keepdims=True)
    for _ in range(invalid):
        t, s = rng.integers(T), rng.integers(topk)
        ids[t, s] = -1 if rng.random() < 0.5 else E + int(rng.integers(3))
    return ids, w


@pytest.mark.parametrize("T,topk,E,hidden,inter,Ks,cb", [
    (1, 8, 16, 256, 256, (3, 3, 3), 1),
    (1, 4, 8, 512, 384, (4, 4, 4), 2),
    (4, 2, 8, 256, 256, (2, 2, 2), 1),
    (7, 3, 6, 256, 128, (3, 4, 2), 1),      # per-projection K (gate != up -> two gate/up launches)
    (16, 8, 32, 512, 256, (3, 3, 3), 1),
    (33, 2, 4, 256, 256, (3, 3, 3), 2),     # 33 tokens over 4 experts: > 16 rows per expert
    (80, 2, 2, 256, 128, (2, 2, 2), 1),     # > 64 rows per expert: several row passes
    (5, 2, 4, 256, 256, (3, 3, 3), 0),      # 3INST codebook
])
def test_moe_layer_vs_oracle(T, topk, E, hidden, inter, Ks, cb):
    print(f"case: moe T={T} topk={topk} E={E} h={hidden} i={inter} K={Ks} cb={cb}", flush=True)
    ex = Experts(E, hidden, inter, Ks, cb, seed=T * 7 + E)
    x = make_x(T, hidden, seed=T + 11)
    ids, w = _routing(T, topk, E, seed=T * 3 + topk)
    if cb == 0:
        out = _layer_capi(ex, x, ids, w, cb=0)
    else:
        out = ex.layer(torch.from_numpy(x).cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda())
    torch.cuda.synchronize()
    assert out.shape == (T, hidden) and out.dtype == torch.float16
    check_close(out.float().cpu().numpy(), ex.ref(x, ids, w), f"moe T={T} E={E}")


def _layer_capi(ex, x, ids, w, cb, limit=0.0):
    T, hidden = x.shape
    topk = ids.shape[1]
    xd, idd, wd = (torch.from_numpy(a).cuda() for a in (x, ids, w))
    out = torch.empty((T, hidden), dtype=torch.float16, device="cuda")
    L = _lib.lib()
    need = int(L.exl3_moe_workspace_size(T, topk, ex.E, hidden, ex.inter))
    ws = ops.workspace(xd.device, need)
    rc = L.exl3_moe_layer(xd.data_ptr(), idd.data_ptr(), wd.data_ptr(), *[t.data_ptr() for t in ex.tables], ex.E,
                          out.data_ptr(), T, topk, hidden, ex.inter, *ex.Ks, cb, limit, ws.data_ptr(), ws.numel(),
                          torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "exl3_moe_layer")
    return out


def test_moe_invalid_ids_are_skipped():
    T, topk, E = 6, 4, 8
    ex = Experts(E, 256, 256, (3, 3, 3), 1, seed=5)
    x = make_x(T, 256, seed=3)
    ids, w = _routing(T, topk, E, seed=9, invalid=5)
    ids[2, :] = -1  # a token with no valid expert -> zero row
    out = ex.layer(torch.from_numpy(x).cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda())
    o = out.float().cpu().numpy()
    assert np.all(o[2] == 0.0)
    check_close(o, ex.ref(x, ids, w), "moe invalid ids")


def test_moe_swiglu_limit():
    """Gate values here have rms ~5, so L = 2 clamps many of them.  (A much
    smaller L on much larger activations is ill-conditioned for any
    implementation: there the reference's own RNE kernels and RTZ host dequant
    differ by more than the bar, because the clamp turns fp16-level error of
    large gate values into O(1) output error.)"""
    T, topk, E = 3, 4, 8
    ex = Experts(E, 256, 256, (4, 4, 4), 1, seed=6)
    x = make_x(T, 256, seed=4)
    ids, w = _routing(T, topk, E, seed=10)
    lim = 2.0
    out = ex.layer(torch.from_numpy(x).cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda(), lim)
    o = out.float().cpu().numpy()
    check_close(o, ex.ref(x, ids, w, lim), "moe limit")
    unclamped = ex.ref(x, ids, w)
    clamped = ex.ref(x, ids, w, lim)
    rms = float(np.sqrt(np.mean(clamped ** 2)))
    assert np.max(np.abs(unclamped - clamped)) > 0.1 * rms  # the clamp matters at this scale


def test_moe_deterministic_and_graph_capturable():
    T, topk, E = 16, 8, 32
    ex = Experts(E, 512, 256, (3, 3, 3), 1, seed=8)
    x = make_x(T, 512, seed=5)
    ids, w = _routing(T, topk, E, seed=12)
    xd, idd, wd = (torch.from_numpy(a).cuda() for a in (x, ids, w))
    a = ex.layer(xd, idd, wd)
    b = ex.layer(xd, idd, wd)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    # capture into a HIP graph; replays interleaved with eager work must match
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ex.layer(xd, idd, wd)  # warm the per-stream workspace outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            gout = ex.layer(xd, idd, wd)
    torch.cuda.synchronize()
    for r in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(gout, a), f"graph replay {r} differs from eager"
        ex.layer(xd, idd, wd)  # eager call on the default stream between replays
        torch.cuda.synchronize()
    # routing changes between replays are picked up (ids read on device)
    ids2, w2 = _routing(T, topk, E, seed=13)
    idd.copy_(torch.from_numpy(ids2))
    wd.copy_(torch.from_numpy(w2))
    g.replay()
    torch.cuda.synchronize()
    check_close(gout.float().cpu().numpy(), ex.ref(x, ids2, w2), "moe graph new routing")


def test_p2b_fused_moe_op():
    """torch op with the reference schema: one token, fp16 routing weights, out overwritten."""
    E, hidden, inter, topk = 12, 512, 256, 6
    ex = Experts(E, hidden, inter, (2, 2, 2), 1, seed=21)
    x = make_x(1, hidden, seed=8)
    ids, w = _routing(1, topk, E, seed=14)
    w16 = w.astype(np.float16)
    xd = torch.from_numpy(x).cuda()
    out = torch.full_like(xd, 7.0)
    ops.p2b_fused_moe_impl(xd, out, *ex.tables, torch.from_numpy(ids[0]).cuda(), torch.from_numpy(w16[0]).cuda(),
                           2, 2, 2, True, intermediate_size=inter, swiglu_limit=0.0)
    torch.cuda.synchronize()
    check_close(out.float().cpu().numpy(), ex.ref(x, ids, w16.astype(np.float32)), "p2b_fused_moe")
    # through torch.ops with the reference's default intermediate size (2048)
    ex2 = Experts(4, 256, 2048, (3, 3, 3), 1, seed=22)
    x2 = make_x(1, 256, seed=9)
    ids2, w2 = _routing(1, 2, 4, seed=15)
    w2h = w2.astype(np.float16)
    x2d = torch.from_numpy(x2).cuda()
    out2 = torch.empty_like(x2d)
    torch.ops.sglang_exl3.p2b_fused_moe(x2d, out2, *ex2.tables, torch.from_numpy(ids2[0]).cuda(),
                                        torch.from_numpy(w2h[0]).cuda(), 3, 3, 3, True)
    torch.cuda.synchronize()
    check_close(out2.float().cpu().numpy(), ex2.ref(x2, ids2, w2h.astype(np.float32)), "p2b_fused_moe op")


def test_moe_cfg4_batch16():
    """Headline MoE shape (E=128, top-8, hidden 2048, inter 768, K=3, MCG) at B=16."""
    T, topk, E = 16, 8, 128
    ex = Experts(E, 2048, 768, (3, 3, 3), 1, seed=44)
    x = make_x(T, 2048, seed=16)
    ids, w = _routing(T, topk, E, seed=17)
    out = ex.layer(torch.from_numpy(x).cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda())
    torch.cuda.synchronize()
    check_close(out.float().cpu().numpy(), ex.ref(x, ids, w), "moe cfg4 B=16")


@pytest.mark.parametrize("T,topk,E,cb,invalid", [(2, 4, 8, 1, 0), (9, 4, 8, 2, 3), (33, 2, 4, 1, 0), (12, 6, 16, 0, 2)])
@pytest.mark.parametrize("rot_tokens", [1, 100000])
def test_moe_rotation_pass(T, topk, E, cb, invalid, rot_tokens, monkeypatch):
    """Gate/up input rows rotated once per call in a pass of their own (threshold 1) or by every
    GEMV item (threshold above T): both against the oracle, with skipped slots."""
    print(f"case: moe rotation pass T={T} topk={topk} E={E} cb={cb} rot_tokens={rot_tokens}", flush=True)
    monkeypatch.setenv("EXL3_MOE_ROT_TOKENS", str(rot_tokens))
    ex = Experts(E, 512, 256, (3, 3, 3), cb, seed=80 + T + E)
    x = make_x(T, 512, seed=81 + T)
    ids, w = _routing(T, topk, E, seed=82 + T, invalid=invalid)
    out = _layer_capi(ex, x, ids, w, cb=cb)
    torch.cuda.synchronize()
    check_close(out.float().cpu().numpy(), ex.ref(x, ids, w), f"moe rotation pass T={T}")


@pytest.mark.parametrize("T,topk,E,fc_tokens", [(6, 4, 8, 0), (6, 4, 8, 16), (33, 2, 4, 100), (20, 8, 16, 100)])
def test_moe_fused_combine(T, topk, E, fc_tokens, monkeypatch):
    """Weighted combine in the down pass (fixed-point accumulators, fc_tokens >= T) or in its own
    kernel (fc_tokens < T): both against the oracle, a token without valid slots gives a zero row,
    and repeated calls give the same bits (the accumulators are left zero)."""
    print(f"case: moe fused combine T={T} topk={topk} E={E} fc_tokens={fc_tokens}", flush=True)
    monkeypatch.setenv("EXL3_MOE_FC_TOKENS", str(fc_tokens))
    ex = Experts(E, 256, 256, (3, 3, 3), 1, seed=90 + T)
    x = make_x(T, 256, seed=91 + T)
    ids, w = _routing(T, topk, E, seed=92 + T, invalid=3)
    ids[T // 2, :] = -1
    a = _layer_capi(ex, x, ids, w, cb=1)
    b = _layer_capi(ex, x, ids, w, cb=1)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    o = a.float().cpu().numpy()
    assert np.all(o[T // 2] == 0.0)
    check_close(o, ex.ref(x, ids, w), f"moe fused combine T={T}")


@pytest.mark.parametrize("direct", ["0", "1"])
@pytest.mark.parametrize("topk,E,invalid,fc_tokens", [(8, 16, 0, 16), (6, 8, 2, 16), (4, 8, 4, 16), (8, 16, 3, 0)])
def test_moe_one_token_direct_routing(topk, E, invalid, fc_tokens, direct, monkeypatch):
    """One token: the GEMV workgroups map units to slots themselves (no routing kernel) or use the
    routing kernel; skipped slots, a token with no valid slot (zero row) and both combine paths."""
    print(f"case: moe one token topk={topk} E={E} invalid={invalid} fc_tokens={fc_tokens} direct={direct}",
          flush=True)
    monkeypatch.setenv("EXL3_MOE_DIRECT", direct)
    monkeypatch.setenv("EXL3_MOE_FC_TOKENS", str(fc_tokens))
    ex = Experts(E, 256, 384, (3, 3, 3), 1, seed=70 + topk + invalid)
    x = make_x(1, 256, seed=71 + topk)
    ids, w = _routing(1, topk, E, seed=72 + topk + invalid)
    ids[0, :invalid] = [-1 if j % 2 else E + j for j in range(invalid)]
    out = _layer_capi(ex, x, ids, w, cb=1)
    torch.cuda.synchronize()
    o = out.float().cpu().numpy()
    if invalid == topk:
        assert np.all(o == 0.0)
    else:
        check_close(o, ex.ref(x, ids, w), f"moe one token direct={direct}")


@pytest.mark.parametrize("E,hidden,inter,K,cb,topk,invalid,fc_tokens", [
    (16, 256, 384, 3, 1, 8, 0, 16),
    (8, 512, 256, 2, 2, 6, 2, 16),
    (8, 256, 768, 4, 0, 4, 1, 0),
    (8, 256, 256, 3, 1, 4, 4, 16),       # no valid slot: zero row
    (128, 2048, 768, 3, 1, 8, 0, 16),    # headline MoE shape
    (32, 1024, 1536, 5, 2, 8, 3, 16),
])
def test_moe_one_token_fused_launch(E, hidden, inter, K, cb, topk, invalid, fc_tokens, monkeypatch):
    """One token with one K: gate/up and down in one launch (opt-in, EXL3_MOE_FUSED=1), the down
    items waiting on readiness flags of the h blocks.  Same bits as the two-launch path with the
    same per-block hand-off (EXL3_MOE_FUSED=0, EXL3_MOE_FXS=0), repeated calls agree (flags and
    counters are left clear), and against the oracle."""
    print(f"case: moe fused one token E={E} h={hidden} i={inter} K={K} cb={cb} topk={topk} invalid={invalid} "
          f"fc_tokens={fc_tokens}", flush=True)
    monkeypatch.setenv("EXL3_MOE_FC_TOKENS", str(fc_tokens))
    monkeypatch.setenv("EXL3_MOE_FXS", "0")  # the two launches with the fused launch's per-block hand-off
    ex = Experts(E, hidden, inter, (K, K, K), cb, seed=150 + E + K)
    x = make_x(1, hidden, seed=151 + K)
    ids, w = _routing(1, topk, E, seed=152 + invalid)
    ids[0, :invalid] = [-1 if j % 2 else E + j for j in range(invalid)]
    outs = {}
    for fused in ("0", "1", "1"):
        monkeypatch.setenv("EXL3_MOE_FUSED", fused)
        o = _layer_capi(ex, x, ids, w, cb=cb)
        torch.cuda.synchronize()
        if fused in outs:
            assert torch.equal(o, outs[fused]), "repeated fused call differs"
        outs[fused] = o
    assert torch.equal(outs["0"], outs["1"]), "fused launch differs from the two launches"
    o = outs["1"].float().cpu().numpy()
    if invalid == topk:
        assert np.all(o == 0.0)
    else:
        check_close(o, ex.ref(x, ids, w), f"moe fused one token E={E}")


@pytest.mark.parametrize("E,hidden,inter,K,cb,topk,invalid,gu_ns", [
    (16, 256, 384, 3, 1, 8, 0, 4),
    (8, 512, 256, 2, 2, 6, 2, 8),
    (8, 256, 768, 4, 0, 4, 1, 2),
    (8, 256, 256, 3, 1, 4, 4, 4),        # no valid slot: zero row
    (128, 2048, 768, 3, 1, 8, 0, 8),     # headline MoE shape
    (32, 1024, 1536, 5, 2, 8, 3, 8),
])
def test_moe_one_token_fused_split_fixed_point(E, hidden, inter, K, cb, topk, invalid, gu_ns, monkeypatch):
    """One token in one launch with the split fixed-point gate/up (EXL3_MOE_FUSED=1, EXL3_MOE_GFX
    on): down items wait until the 2 S gate/up items of each h block have added (and stored the
    elements they completed).  Same bits as the two launches with the same gate/up items, repeated
    calls agree (readiness counts and accumulators are left clear), and against the oracle."""
    print(f"case: moe fused gfx one token E={E} h={hidden} i={inter} K={K} cb={cb} topk={topk} invalid={invalid} "
          f"gu_ns={gu_ns}", flush=True)
    monkeypatch.setenv("EXL3_MOE_GFX_GU_NSTEPS", str(gu_ns))
    ex = Experts(E, hidden, inter, (K, K, K), cb, seed=210 + E + K)
    x = make_x(1, hidden, seed=211 + K)
    ids, w = _routing(1, topk, E, seed=212 + invalid)
    ids[0, :invalid] = [-1 if j % 2 else E + j for j in range(invalid)]
    outs = {}
    for fused in ("0", "1", "1"):
        monkeypatch.setenv("EXL3_MOE_FUSED", fused)
        o = _layer_capi(ex, x, ids, w, cb=cb)
        torch.cuda.synchronize()
        if fused in outs:
            assert torch.equal(o, outs[fused]), "repeated fused call differs"
        outs[fused] = o
    assert torch.equal(outs["0"], outs["1"]), "fused launch differs from the two launches"
    o = outs["1"].float().cpu().numpy()
    if invalid == topk:
        assert np.all(o == 0.0)
    else:
        check_close(o, ex.ref(x, ids, w), f"moe fused gfx one token E={E}")


@pytest.mark.parametrize("T,topk,E,hidden,inter,K,cb,invalid", [
    (2, 8, 128, 2048, 768, 3, 1, 0),      # split fixed-point gate/up, 4-step down items
    (3, 4, 16, 512, 512, 2, 2, 1),        # mul1, 8-step down items
    (16, 8, 128, 2048, 768, 3, 1, 0),     # headline shape: fused combine, 12-step down items
    (16, 8, 32, 1024, 1536, 4, 0, 3),     # 3INST
    (40, 2, 4, 512, 512, 3, 1, 2),        # more than 16 rows per expert: several units per expert
    (64, 8, 128, 2048, 768, 3, 1, 0),     # separate combine, per-block hand-off of the down pass
])
def test_moe_routed_fused_launch(T, topk, E, hidden, inter, K, cb, invalid, monkeypatch):
    """A routed batch with gate/up and down in one launch after the routing launch (opt-in,
    EXL3_MOE_FUSED_ROUTED=1, which plans 4- or 8-step down items): same bits as the separate gate/up
    and down launches with the same items, repeated calls agree (readiness counts, hand-off counters
    and accumulators are left clear), and against the oracle."""
    print(f"case: moe fused routed T={T} topk={topk} E={E} h={hidden} i={inter} K={K} cb={cb} invalid={invalid}",
          flush=True)
    monkeypatch.setenv("EXL3_MOE_DN_NSTEPS", "4" if inter % 512 else "8")  # the fused pass's down items
    ex = Experts(E, hidden, inter, (K, K, K), cb, seed=230 + T + E)
    x = make_x(T, hidden, seed=231 + T)
    ids, w = _routing(T, topk, E, seed=232 + T, invalid=invalid)
    outs = {}
    for fused in ("0", "1", "1"):
        monkeypatch.setenv("EXL3_MOE_FUSED_ROUTED", fused)
        o = _layer_capi(ex, x, ids, w, cb=cb)
        torch.cuda.synchronize()
        if fused in outs:
            assert torch.equal(o, outs[fused]), "repeated fused routed call differs"
        outs[fused] = o
    assert torch.equal(outs["0"], outs["1"]), "fused routed launch differs from the separate launches"
    check_close(outs["1"].float().cpu().numpy(), ex.ref(x, ids, w), f"moe fused routed T={T}")


def test_moe_routed_fused_graph(monkeypatch):
    """The routed one-launch gate/up + down pass captured in a HIP graph: replays interleaved with
    eager calls match the eager result, and a routing change between replays is picked up."""
    monkeypatch.setenv("EXL3_MOE_FUSED_ROUTED", "1")
    T, E, hidden, inter, topk = 12, 32, 512, 768, 8
    ex = Experts(E, hidden, inter, (3, 3, 3), 1, seed=240)
    x = make_x(T, hidden, seed=241)
    ids, w = _routing(T, topk, E, seed=242)
    xd, idd, wd = (torch.from_numpy(a).cuda() for a in (x, ids, w))
    a = ex.layer(xd, idd, wd)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ex.layer(xd, idd, wd)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            gout = ex.layer(xd, idd, wd)
    torch.cuda.synchronize()
    for r in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(gout, a), f"graph replay {r} differs from eager"
        ex.layer(xd, idd, wd)
        torch.cuda.synchronize()
    ids2, w2 = _routing(T, topk, E, seed=243, invalid=3)
    idd.copy_(torch.from_numpy(ids2))
    wd.copy_(torch.from_numpy(w2))
    g.replay()
    torch.cuda.synchronize()
    check_close(gout.float().cpu().numpy(), ex.ref(x, ids2, w2), "moe fused routed graph new routing")


def test_moe_one_token_fused_graph(monkeypatch):
    """The fused one-token launch captured in a HIP graph: replays interleaved with eager calls
    match the eager result, and a routing change between replays is picked up."""
    monkeypatch.setenv("EXL3_MOE_FUSED", "1")
    E, hidden, inter, topk = 32, 512, 768, 8
    ex = Experts(E, hidden, inter, (3, 3, 3), 1, seed=160)
    x = make_x(1, hidden, seed=161)
    ids, w = _routing(1, topk, E, seed=162)
    xd, idd, wd = (torch.from_numpy(a).cuda() for a in (x, ids, w))
    a = ex.layer(xd, idd, wd)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ex.layer(xd, idd, wd)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            gout = ex.layer(xd, idd, wd)
    torch.cuda.synchronize()
    for r in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(gout, a), f"graph replay {r} differs from eager"
        ex.layer(xd, idd, wd)
        torch.cuda.synchronize()
    ids2, w2 = _routing(1, topk, E, seed=163)
    ids2[0, 3] = -1
    idd.copy_(torch.from_numpy(ids2))
    wd.copy_(torch.from_numpy(w2))
    g.replay()
    torch.cuda.synchronize()
    check_close(gout.float().cpu().numpy(), ex.ref(x, ids2, w2), "moe fused graph new routing")


@pytest.mark.parametrize("E,hidden,inter,Ks,cb,topk,invalid,gu_ns,limit", [
    (16, 256, 384, (3, 3, 3), 1, 8, 0, 4, 0.0),
    (8, 512, 256, (2, 2, 2), 2, 6, 2, 2, 0.0),       # mul1: per-split row sums in the fixed-point adds
    (8, 256, 768, (4, 4, 4), 0, 4, 1, 4, 0.0),       # 3INST
    (8, 256, 256, (3, 3, 3), 1, 4, 4, 4, 0.0),       # no valid slot: zero row
    (128, 2048, 768, (3, 3, 3), 1, 8, 0, 4, 0.0),    # headline MoE shape
    (128, 2048, 768, (3, 3, 3), 1, 8, 0, 2, 0.0),    # 16 splits
    (32, 1024, 1536, (5, 5, 5), 2, 8, 3, 8, 0.0),
    (8, 512, 384, (3, 4, 2), 1, 4, 0, 4, 0.0),       # gate != up: two gate/up launches
    (8, 256, 256, (4, 4, 4), 1, 4, 0, 4, 2.0),       # SwiGLU clamp in the down staging
])
def test_moe_one_token_split_fixed_point_gate_up(E, hidden, inter, Ks, cb, topk, invalid, gu_ns, limit, monkeypatch):
    """One token, two launches (EXL3_MOE_GFX, default on): gate/up items add their rotated, scaled
    partial rows into fixed-point accumulators, each element's completing add writes the fp16 gate
    or up value, and the down pass stages the SwiGLU from them.  Against the oracle, against the
    partial-row hand-off (EXL3_MOE_GFX=0) within the same bar, repeated calls bit-identical (the
    accumulators are left clear), skipped slots and a token without valid slots."""
    print(f"case: moe gfx one token E={E} h={hidden} i={inter} K={Ks} cb={cb} topk={topk} invalid={invalid} "
          f"gu_ns={gu_ns} limit={limit}", flush=True)
    monkeypatch.setenv("EXL3_MOE_GFX_GU_NSTEPS", str(gu_ns))
    ex = Experts(E, hidden, inter, Ks, cb, seed=190 + E + Ks[0])
    x = make_x(1, hidden, seed=191 + Ks[0])
    ids, w = _routing(1, topk, E, seed=192 + invalid)
    ids[0, :invalid] = [-1 if j % 2 else E + j for j in range(invalid)]
    monkeypatch.setenv("EXL3_MOE_GFX", "0")
    base = _layer_capi(ex, x, ids, w, cb=cb, limit=limit)
    monkeypatch.setenv("EXL3_MOE_GFX", "1")
    a = _layer_capi(ex, x, ids, w, cb=cb, limit=limit)
    b = _layer_capi(ex, x, ids, w, cb=cb, limit=limit)
    torch.cuda.synchronize()
    assert torch.equal(a, b), "repeated call differs"
    o = a.float().cpu().numpy()
    if invalid == topk:
        assert np.all(o == 0.0)
        return
    ref = ex.ref(x, ids, w, limit if limit > 0 else float("inf"))
    check_close(o, ref, f"moe gfx one token E={E}")
    check_close(o, base.float().cpu().numpy(), f"moe gfx vs partial-row hand-off E={E}")


@pytest.mark.parametrize("T,topk,E,hidden,inter,Ks,cb,invalid,gu_ns", [
    (2, 8, 16, 256, 384, (3, 3, 3), 1, 0, 4),
    (5, 4, 8, 512, 256, (2, 2, 2), 2, 3, 8),
    (16, 8, 32, 512, 768, (3, 3, 3), 1, 4, 4),
    (16, 8, 128, 2048, 768, (3, 3, 3), 1, 0, 4),    # headline MoE shape
    (9, 6, 8, 256, 256, (4, 3, 2), 0, 2, 2),        # 3INST, gate != up
])
def test_moe_batch_split_fixed_point_gate_up(T, topk, E, hidden, inter, Ks, cb, invalid, gu_ns, monkeypatch):
    """Routed batches with the fused combine: the split fixed-point gate/up pass on the rotated rows
    (EXL3_MOE_GFX) against the oracle and the partial-row hand-off, repeated calls bit-identical, a
    token without valid slots a zero row."""
    print(f"case: moe gfx batch T={T} topk={topk} E={E} h={hidden} i={inter} K={Ks} cb={cb} gu_ns={gu_ns}",
          flush=True)
    monkeypatch.setenv("EXL3_MOE_GFX_GU_NSTEPS", str(gu_ns))
    monkeypatch.setenv("EXL3_MOE_GFX_TOKENS", "16")  # above the default threshold too
    ex = Experts(E, hidden, inter, Ks, cb, seed=200 + T + E)
    x = make_x(T, hidden, seed=201 + T)
    ids, w = _routing(T, topk, E, seed=202 + T, invalid=invalid)
    if T > 2:
        ids[T // 2, :] = -1
    monkeypatch.setenv("EXL3_MOE_GFX", "0")
    base = _layer_capi(ex, x, ids, w, cb=cb)
    monkeypatch.setenv("EXL3_MOE_GFX", "1")
    a = _layer_capi(ex, x, ids, w, cb=cb)
    b = _layer_capi(ex, x, ids, w, cb=cb)
    torch.cuda.synchronize()
    assert torch.equal(a, b), "repeated call differs"
    o = a.float().cpu().numpy()
    if T > 2:
        assert np.all(o[T // 2] == 0.0)
    check_close(o, ex.ref(x, ids, w), f"moe gfx batch T={T}")
    check_close(o, base.float().cpu().numpy(), f"moe gfx batch vs partial-row hand-off T={T}")


def test_moe_one_token_split_fixed_point_graph():
    """The split fixed-point gate/up path captured in a HIP graph: replays interleaved with eager
    calls match the eager result, and a routing change between replays is picked up."""
    E, hidden, inter, topk = 32, 512, 768, 8
    ex = Experts(E, hidden, inter, (3, 3, 3), 1, seed=195)
    x = make_x(1, hidden, seed=196)
    ids, w = _routing(1, topk, E, seed=197)
    xd, idd, wd = (torch.from_numpy(a).cuda() for a in (x, ids, w))
    a = ex.layer(xd, idd, wd)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ex.layer(xd, idd, wd)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            gout = ex.layer(xd, idd, wd)
    torch.cuda.synchronize()
    for r in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(gout, a), f"graph replay {r} differs from eager"
        ex.layer(xd, idd, wd)
        torch.cuda.synchronize()
    ids2, w2 = _routing(1, topk, E, seed=198)
    ids2[0, 5] = E + 1
    idd.copy_(torch.from_numpy(ids2))
    wd.copy_(torch.from_numpy(w2))
    g.replay()
    torch.cuda.synchronize()
    check_close(gout.float().cpu().numpy(), ex.ref(x, ids2, w2), "moe gfx graph new routing")


@pytest.mark.parametrize("T,topk,E,hidden,inter,K,cb,invalid", [
    (1, 8, 16, 256, 768, 3, 1, 0), (1, 6, 8, 512, 384, 4, 2, 2), (5, 4, 8, 256, 1536, 3, 0, 3),
    (16, 8, 32, 512, 768, 2, 1, 4), (12, 2, 4, 256, 256, 5, 2, 0),
])
def test_moe_split_fixed_point_combine(T, topk, E, hidden, inter, K, cb, invalid, monkeypatch):
    """Fused combine with one round trip per split (EXL3_MOE_FXS, default on): every k-split item
    adds its rotated, scaled partial rows into the output accumulators.  Against the oracle, against
    the per-column-block hand-off (EXL3_MOE_FXS=0) within the same bar, repeated calls bit-identical,
    a token without valid slots a zero row."""
    print(f"case: moe split fixed-point T={T} topk={topk} E={E} h={hidden} i={inter} K={K} cb={cb}", flush=True)
    ex = Experts(E, hidden, inter, (K, K, K), cb, seed=170 + T + K)
    x = make_x(T, hidden, seed=171 + T)
    ids, w = _routing(T, topk, E, seed=172 + T, invalid=invalid)
    if T > 2:
        ids[T // 2, :] = -1
    monkeypatch.setenv("EXL3_MOE_FXS", "0")
    base = _layer_capi(ex, x, ids, w, cb=cb)
    monkeypatch.setenv("EXL3_MOE_FXS", "1")
    a = _layer_capi(ex, x, ids, w, cb=cb)
    b = _layer_capi(ex, x, ids, w, cb=cb)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    o = a.float().cpu().numpy()
    if T > 2:
        assert np.all(o[T // 2] == 0.0)
    ref = ex.ref(x, ids, w)
    check_close(o, ref, f"moe split fixed-point T={T}")
    check_close(o, base.float().cpu().numpy(), f"moe split fixed-point vs hand-off T={T}")


@pytest.mark.parametrize("T,inter,fc_tokens", [(20, 768, 100), (20, 1536, 0), (3, 768, 16)])
def test_moe_down_twelve_step_items(T, inter, fc_tokens, monkeypatch):
    """Down pass with 12-step items (48 k-slices: one split at inter 768, two at 1536), forced
    by env, with either combine path."""
    print(f"case: moe down 12-step items T={T} inter={inter} fc_tokens={fc_tokens}", flush=True)
    monkeypatch.setenv("EXL3_MOE_DN_NSTEPS", "12")
    monkeypatch.setenv("EXL3_MOE_FC_TOKENS", str(fc_tokens))
    E, topk = 8, 4
    ex = Experts(E, 256, inter, (3, 3, 3), 1, seed=60 + T)
    x = make_x(T, 256, seed=61 + T)
    ids, w = _routing(T, topk, E, seed=62 + T, invalid=2)
    out = _layer_capi(ex, x, ids, w, cb=1)
    torch.cuda.synchronize()
    check_close(out.float().cpu().numpy(), ex.ref(x, ids, w), f"moe down 12 steps T={T} inter={inter}")


def test_moe_rejects_bad_arguments():
    ex = Experts(2, 256, 128, (2, 2, 2), 1, seed=1)
    x = torch.zeros((1, 200), dtype=torch.float16, device="cuda")
    ids = torch.zeros((1, 1), dtype=torch.int32, device="cuda")
    w = torch.ones((1, 1), dtype=torch.float32, device="cuda")
    with pytest.raises(RuntimeError, match="multiples of 128"):
        ex.layer(x, ids, w)
    with pytest.raises(RuntimeError, match="K"):
        torch.ops.sglang_exl3.exl3_moe_layer(torch.zeros((1, 256), dtype=torch.float16, device="cuda"), ids, w,
                                             *ex.tables, 9, 2, 2, True, 128, 0.0)


# ------------------------------------------------------------- prefill path
#
# Batches whose experts get many rows each (or more than 8192 routed rows) run
# the prefill pipeline: device-side sort into 64/128-row tiles, one rotation
# pass, the grouped MFMA GEMM for gate, up (+ SwiGLU + down rotation) and down,
# then the slot-ordered combine.  EXL3_MOE_PREFILL=1 forces it for small cases.


@pytest.mark.parametrize("T,topk,E,hidden,inter,Ks,cb,invalid", [
    (40, 4, 8, 256, 256, (3, 3, 3), 1, 0),     # ~20 rows per expert: 64-row tiles
    (300, 2, 4, 256, 128, (2, 3, 4), 2, 3),    # ~150 rows per expert: several 128-row tiles; per-projection K
    (64, 8, 16, 512, 384, (4, 4, 4), 0, 5),    # 3INST codebook, invalid ids
    (1, 3, 4, 256, 256, (3, 3, 3), 1, 0),      # a single token through the prefill pipeline
])
def test_moe_prefill_path_vs_oracle(T, topk, E, hidden, inter, Ks, cb, invalid, monkeypatch):
    monkeypatch.setenv("EXL3_MOE_PREFILL", "1")
    print(f"case: moe prefill T={T} topk={topk} E={E} h={hidden} i={inter} K={Ks} cb={cb}", flush=True)
    ex = Experts(E, hidden, inter, Ks, cb, seed=T + 3 * E)
    x = make_x(T, hidden, seed=T + 1)
    ids, w = _routing(T, topk, E, seed=T * 5 + topk, invalid=invalid)
    out = _layer_capi(ex, x, ids, w, cb=cb)
    torch.cuda.synchronize()
    check_close(out.float().cpu().numpy(), ex.ref(x, ids, w), f"moe prefill T={T} E={E}")


def test_moe_prefill_swiglu_limit(monkeypatch):
    monkeypatch.setenv("EXL3_MOE_PREFILL", "1")
    T, topk, E = 48, 2, 4
    ex = Experts(E, 256, 256, (3, 3, 3), 1, seed=21)
    x = (make_x(T, 256, seed=22).astype(np.float32) * 2).astype(np.float16)
    ids, w = _routing(T, topk, E, seed=23)
    out = _layer_capi(ex, x, ids, w, cb=1, limit=2.0)
    torch.cuda.synchronize()
    check_close(out.float().cpu().numpy(), ex.ref(x, ids, w, limit=2.0), "moe prefill limit")


def test_moe_prefill_token_chunks_vs_oracle_subset():
    """16800 routed rows: above one pipeline pass (16384), so two token chunks; checked on 64
    seeded tokens from both chunks (tokens are independent)."""
    T, topk, E, hidden, inter = 2100, 8, 32, 256, 128
    ex = Experts(E, hidden, inter, (3, 3, 3), 1, seed=31)
    x = make_x(T, hidden, seed=32)
    ids, w = _routing(T, topk, E, seed=33, invalid=40)
    out = ex.layer(torch.from_numpy(x).cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda())
    torch.cuda.synchronize()
    sel = np.sort(np.concatenate([np.random.default_rng(34).choice(2048, 48, replace=False),
                                  2048 + np.arange(16) * 3]))
    check_close(out.float().cpu().numpy()[sel], ex.ref(x[sel], ids[sel], w[sel]), "moe prefill chunks")


def test_moe_prefill_graph_capturable(monkeypatch):
    monkeypatch.setenv("EXL3_MOE_PREFILL", "1")
    T, topk, E = 96, 4, 8
    ex = Experts(E, 256, 256, (3, 3, 3), 2, seed=41)
    x = make_x(T, 256, seed=42)
    ids, w = _routing(T, topk, E, seed=43)
    xd, idd, wd = (torch.from_numpy(a).cuda() for a in (x, ids, w))
    a = ex.layer(xd, idd, wd)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ex.layer(xd, idd, wd)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            gout = ex.layer(xd, idd, wd)
    torch.cuda.synchronize()
    for r in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(gout, a), f"prefill graph replay {r} differs from eager"
        ex.layer(xd, idd, wd)
        torch.cuda.synchronize()
    ids2, w2 = _routing(T, topk, E, seed=44)
    idd.copy_(torch.from_numpy(ids2))
    wd.copy_(torch.from_numpy(w2))
    g.replay()
    torch.cuda.synchronize()
    check_close(gout.float().cpu().numpy(), ex.ref(x, ids2, w2), "moe prefill graph new routing")


def test_moe_prefill_and_decode_paths_agree(monkeypatch):
    """The same layer through both pipelines (decode: 16-row GEMV units; prefill: MFMA tiles)."""
    T, topk, E = 64, 4, 8
    ex = Experts(E, 256, 256, (3, 3, 3), 1, seed=51)
    x = make_x(T, 256, seed=52)
    ids, w = _routing(T, topk, E, seed=53)
    outs = {}
    for mode in ("0", "1"):
        monkeypatch.setenv("EXL3_MOE_PREFILL", mode)
        outs[mode] = _layer_capi(ex, x, ids, w, cb=1).float().cpu().numpy()
    ref = ex.ref(x, ids, w)
    check_close(outs["0"], ref, "decode path")
    check_close(outs["1"], ref, "prefill path")


@pytest.mark.parametrize("T,E,hidden,inter,K,cb", [
    (16, 128, 2048, 768, 3, 1),    # uniform routing: the device groups 2 column blocks, the planner 1
    (4, 64, 4096, 1536, 2, 2),     # 8 gate/up splits: split fixed-point gate/up at 4 tokens, 4-block groups
])
def test_moe_column_grouping_keeps_bits(T, E, hidden, inter, K, cb, monkeypatch):
    """The column blocks per item of a routed pass (chosen on the device from the routed unit
    count, or forced with EXL3_MOE_BPI) only move work between workgroups: every grouping gives the
    same bits, and the result matches the oracle."""
    print(f"case: moe column grouping T={T} E={E} h={hidden} i={inter} K={K} cb={cb}", flush=True)
    ex = Experts(E, hidden, inter, (K, K, K), cb, seed=250 + T)
    x = make_x(T, hidden, seed=251 + T)
    ids, w = _routing(T, 8, E, seed=252 + T)
    outs = []
    for dyn, bpi in (("1", None), ("0", None), ("0", "2"), ("0", "3")):
        monkeypatch.setenv("EXL3_MOE_BPI_DYN", dyn)
        if bpi is None:
            monkeypatch.delenv("EXL3_MOE_BPI", raising=False)
        else:
            monkeypatch.setenv("EXL3_MOE_BPI", bpi)
        outs.append(_layer_capi(ex, x, ids, w, cb=cb))
        torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o, outs[0]), "column grouping changed the result"
    check_close(outs[0].float().cpu().numpy(), ex.ref(x, ids, w), f"moe column grouping T={T}")
