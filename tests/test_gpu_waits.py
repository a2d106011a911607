"""Bounded waits that give up are reported, not silent.

Two kernels wait inside a launch: the second k-half of a wide-tile GEMM tail
tile waits for the first half's partial tile, and a down item of the
one-launch MoE passes (one token, EXL3_MOE_FUSED=1; routed batches,
EXL3_MOE_FUSED_ROUTED=1) waits for the h blocks the gate/up items publish.  Both waits are bounded so that every wave exits; a
wait that gives up sets a bit of the workspace status word, which
exl3_workspace_status / ops.check_waits() report.

The tests make a wait give up from the host: EXL3_WAIT_POLLS=0 gives every
bounded wait a budget of zero polls, so it gives up at once (the kernels then
read hand-off buffers that may not be written yet: in-bounds workspace memory,
wrong values, every kernel exits normally).  check_waits() must raise, zero the
workspace, and the next call with the default budget must give the clean result.
"""

import ctypes

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


def test_workspace_status_starts_clear_and_capi_checks_arguments():
    ws = torch.zeros(256 * 1024, dtype=torch.uint8, device="cuda")
    st = ctypes.c_int32(-1)
    L = _lib.lib()
    assert L.exl3_workspace_status(ws.data_ptr(), ws.numel(), ctypes.byref(st), None) == _lib.EXL3_OK
    assert st.value == 0
    assert L.exl3_workspace_status(ws.data_ptr(), 1024, ctypes.byref(st), None) == _lib.EXL3_ERR_ARG
    assert L.exl3_workspace_status(None, ws.numel(), ctypes.byref(st), None) == _lib.EXL3_ERR_ARG
    ops.check_waits()


def test_fat_tail_wait_that_gives_up_is_reported(monkeypatch):
    """Gate/up SwiGLU at m=300 takes the wide-tile kernel, whose 4 tiles all run as
    tail-split k-halves (k=256: 4 steps)."""
    m, k, n, K, cb = 300, 256, 256, 3, 1
    print(f"case: fat tail wait m={m} k={k} n={n} K={K} cb={cb}", flush=True)
    tg, su, sg = make_weight(k, n, K, seed=501)
    tu, _, sv_u = make_weight(k, n, K, seed=502)
    scale = np.float32(4.0 / np.sqrt(k))
    sg = (sg.astype(np.float32) * scale).astype(np.float16)
    sv_u = (sv_u.astype(np.float32) * scale).astype(np.float16)
    x = make_x(m, k, seed=503)
    d = [torch.from_numpy(a).cuda() for a in (x, su, tg, sg, tu, sv_u)]

    def run():
        out = torch.ops.sglang_exl3.exl3_gate_up_swiglu(*d, K, cb, 0.0)
        torch.cuda.synchronize()
        return out

    clean = run()
    ops.check_waits()
    monkeypatch.setenv("EXL3_WAIT_POLLS", "0")
    run()
    with pytest.raises(RuntimeError, match="tail tile"):
        ops.check_waits()
    monkeypatch.delenv("EXL3_WAIT_POLLS")
    again = run()
    ops.check_waits()
    assert torch.equal(again, clean)
    g = oracle.matmul(x, oracle.dequant(tg, su, sg, K, cb, rtz=True))
    u = oracle.matmul(x, oracle.dequant(tu, su, sv_u, K, cb, rtz=True))
    check_close(again.float().cpu().numpy(), oracle.swiglu(g, u, float("inf")), "gate_up after a reported wait")


def test_moe_fused_wait_that_gives_up_is_reported(monkeypatch):
    """One token, one K, the one-launch MoE layer: with a zero poll budget the down
    items stop waiting at once; check_waits() reports it, and the next call matches
    the two-launch path bit for bit."""
    E, hidden, inter, K, cb, topk = 16, 256, 256, 3, 1, 8
    print(f"case: moe fused wait E={E} h={hidden} i={inter} K={K} topk={topk}", flush=True)
    monkeypatch.setenv("EXL3_MOE_FXS", "0")  # the two launches with the fused launch's per-block hand-off
    rng = np.random.default_rng(510)
    tabs = {p: ([], [], []) for p in ("gate", "up", "down")}
    keep = []
    for e in range(E):
        for j, (proj, kk, nn) in enumerate((("gate", hidden, inter), ("up", hidden, inter), ("down", inter, hidden))):
            tr, su, sv = make_weight(kk, nn, K, seed=520 + 3 * e + j)
            sv = (sv.astype(np.float32) * (4.0 / np.sqrt(kk))).astype(np.float16)
            dd = [torch.from_numpy(a).cuda() for a in (tr, su, sv)]
            keep.append(dd)
            for c, t in zip(tabs[proj], dd):
                c.append(t.data_ptr())
    tables = [torch.tensor(c, dtype=torch.int64, device="cuda") for p in ("gate", "up", "down") for c in tabs[p]]
    x = torch.from_numpy(make_x(1, hidden, seed=511)).cuda()
    ids = torch.from_numpy(rng.choice(E, size=(1, topk), replace=False).astype(np.int32)).cuda()
    w = torch.from_numpy((rng.random((1, topk)) + 0.05).astype(np.float32)).cuda()

    def run(fused):
        monkeypatch.setenv("EXL3_MOE_FUSED", fused)
        out = torch.ops.sglang_exl3.exl3_moe_layer(x, ids, w, *tables, K, K, K, cb == 1, inter, 0.0)
        torch.cuda.synchronize()
        return out

    two = run("0")
    ops.check_waits()
    monkeypatch.setenv("EXL3_WAIT_POLLS", "0")
    run("1")
    with pytest.raises(RuntimeError, match="down item"):
        ops.check_waits()
    monkeypatch.delenv("EXL3_WAIT_POLLS")
    again = run("1")
    ops.check_waits()
    assert torch.equal(again, two)
    del keep


def test_moe_routed_fused_wait_that_gives_up_is_reported(monkeypatch):
    """A routed batch in the one-launch gate/up + down pass (EXL3_MOE_FUSED_ROUTED=1): with a
    zero poll budget the down items stop waiting at once; check_waits() reports it, and the next
    call matches the separate launches bit for bit."""
    T, E, hidden, inter, K, cb, topk = 12, 16, 512, 512, 3, 1, 4
    print(f"case: moe fused routed wait T={T} E={E} h={hidden} i={inter} K={K} topk={topk}", flush=True)
    monkeypatch.setenv("EXL3_MOE_DN_NSTEPS", "8")  # the fused pass's down items, for both paths
    rng = np.random.default_rng(530)
    tabs = {p: ([], [], []) for p in ("gate", "up", "down")}
    keep = []
    for e in range(E):
        for j, (proj, kk, nn) in enumerate((("gate", hidden, inter), ("up", hidden, inter), ("down", inter, hidden))):
            tr, su, sv = make_weight(kk, nn, K, seed=540 + 3 * e + j)
            sv = (sv.astype(np.float32) * (4.0 / np.sqrt(kk))).astype(np.float16)
            dd = [torch.from_numpy(a).cuda() for a in (tr, su, sv)]
            keep.append(dd)
            for c, t in zip(tabs[proj], dd):
                c.append(t.data_ptr())
    tables = [torch.tensor(c, dtype=torch.int64, device="cuda") for p in ("gate", "up", "down") for c in tabs[p]]
    x = torch.from_numpy(make_x(T, hidden, seed=531)).cuda()
    ids = torch.from_numpy(np.stack([rng.choice(E, size=topk, replace=False) for _ in range(T)]).astype(np.int32)).cuda()
    w = torch.from_numpy((rng.random((T, topk)) + 0.05).astype(np.float32)).cuda()

    def run(fused):
        monkeypatch.setenv("EXL3_MOE_FUSED_ROUTED", fused)
        out = torch.ops.sglang_exl3.exl3_moe_layer(x, ids, w, *tables, K, K, K, cb == 1, inter, 0.0)
        torch.cuda.synchronize()
        return out

    two = run("0")
    ops.check_waits()
    monkeypatch.setenv("EXL3_WAIT_POLLS", "0")
    run("1")
    with pytest.raises(RuntimeError, match="down item"):
        ops.check_waits()
    monkeypatch.delenv("EXL3_WAIT_POLLS")
    again = run("1")
    ops.check_waits()
    assert torch.equal(again, two)
    del keep
