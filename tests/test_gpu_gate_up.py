"""GPU parity of the fused gate+up SwiGLU op (exl3_gate_up_swiglu) against the
oracle: out = silu(min(x W_g, L)) * clamp(x W_u, -L, L), both weights sharing
the input rotation suh, as the reference's fused gate/up path does
(src/sglang_exl3/exl3.py:1184-1206).  Up to 3 rows the GEMV kernel (gate and
up rounded to fp16 first), up to 160 the narrow MFMA kernel in gate/up mode
(k-splits hand partial tiles to the last split, or up to 16 rows to a finish
launch), above the wide-tile MFMA kernel (fp32 accumulators throughout).  Bar: max-abs-err <= 2e-2 * rms(ref),
cosine >= 0.9999."""

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


def _pair(k, n, K, seed):
    """Gate and up weights with one shared suh (output scale folded into svh)."""
    tg, su, sg = make_weight(k, n, K, seed=seed)
    tu, _, su2 = make_weight(k, n, K, seed=seed + 1)
    scale = np.float32(4.0 / np.sqrt(k))
    sg = (sg.astype(np.float32) * scale).astype(np.float16)
    su2 = (su2.astype(np.float32) * scale).astype(np.float16)
    return tg, su, sg, tu, su2


def _ref(x, tg, su, sg, tu, sv_u, K, cb, limit, rows=None):
    xs = x if rows is None else x[rows]
    g = oracle.matmul(xs, oracle.dequant(tg, su, sg, K, cb, rtz=True))
    u = oracle.matmul(xs, oracle.dequant(tu, su, sv_u, K, cb, rtz=True))
    return oracle.swiglu(g, u, limit)


def _run(x, tg, su, sg, tu, sv_u, K, cb, limit=0.0):
    d = [torch.from_numpy(a).cuda() for a in (x, su, tg, sg, tu, sv_u)]
    out = torch.ops.sglang_exl3.exl3_gate_up_swiglu(*d, K, cb, limit)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("m,k,n,K,cb", [
    (1, 256, 256, 4, 1), (5, 512, 384, 3, 2), (16, 256, 512, 2, 1), (40, 384, 256, 5, 0), (64, 256, 256, 3, 1),
    (65, 512, 256, 4, 1), (300, 256, 384, 3, 2), (520, 1024, 256, 2, 0), (257, 256, 128, 6, 1),
])
def test_gate_up_swiglu_vs_oracle(m, k, n, K, cb):
    print(f"case: gate_up m={m} k={k} n={n} K={K} cb={cb}", flush=True)
    tg, su, sg, tu, sv_u = _pair(k, n, K, seed=m * 7 + K)
    x = make_x(m, k, seed=m + 3)
    out = _run(x, tg, su, sg, tu, sv_u, K, cb)
    assert out.shape == (m, n) and out.dtype == torch.float16
    check_close(out.float().cpu().numpy(), _ref(x, tg, su, sg, tu, sv_u, K, cb, float("inf")), f"gate_up m={m}")


@pytest.mark.parametrize("m,cb", [(5, 2), (13, 0), (40, 1), (100, 2), (150, 0), (160, 1)])
def test_gate_up_split_handoff_ragged_rows(m, cb):
    """The narrow kernel's gate/up k-splits (k = 2048: two splits of 16 steps,
    n = 384: three column blocks per projection) on row counts that leave the
    last row tile partial; bit-identical on a repeat call (the counters reset
    themselves)."""
    k, n, K = 2048, 384, 3
    print(f"case: gate_up split hand-off ragged m={m} cb={cb}", flush=True)
    tg, su, sg, tu, sv_u = _pair(k, n, K, seed=110 + m)
    x = make_x(m, k, seed=111 + m)
    first = _run(x, tg, su, sg, tu, sv_u, K, cb)
    again = _run(x, tg, su, sg, tu, sv_u, K, cb)
    assert torch.equal(first, again), "gate/up split hand-off: repeated calls differ"
    check_close(first.float().cpu().numpy(), _ref(x, tg, su, sg, tu, sv_u, K, cb, float("inf")),
                f"gate_up split hand-off m={m} cb={cb}")


@pytest.mark.parametrize("m,cb,limit", [(6, 2, 0.0), (9, 1, 1.5), (16, 2, 0.0), (16, 0, 2.0)])
def test_gate_up_split_out_finish_matches_in_kernel_handoff(m, cb, limit, monkeypatch):
    """From 6 to 16 rows the narrow gate/up k-splits store their partial tiles and
    a second launch (fat_gu_finish_kernel) finishes every row; its sums and
    epilogue are the in-kernel hand-off's, so both give the same bits
    (EXL3_FAT_SPLIT_OUT=0 keeps the hand-off), also with a clamp and the
    mul1 raw-entry map (cb 2)."""
    k, n, K = 2048, 384, 3
    print(f"case: gate_up split-out finish m={m} cb={cb} limit={limit}", flush=True)
    tg, su, sg, tu, sv_u = _pair(k, n, K, seed=120 + m + cb)
    x = make_x(m, k, seed=121 + m)
    monkeypatch.setenv("EXL3_GATE_UP_GEMV_ROWS", "0")  # the MFMA path at every m
    split = _run(x, tg, su, sg, tu, sv_u, K, cb, limit)
    monkeypatch.setenv("EXL3_FAT_SPLIT_OUT", "0")
    handoff = _run(x, tg, su, sg, tu, sv_u, K, cb, limit)
    assert torch.equal(split.view(torch.int16), handoff.view(torch.int16))
    ref = _ref(x, tg, su, sg, tu, sv_u, K, cb, limit if limit > 0 else float("inf"))
    check_close(split.float().cpu().numpy(), ref, f"gate_up split-out m={m} cb={cb}")


@pytest.mark.parametrize("m", [8, 200])
def test_gate_up_swiglu_limit(m):
    """The clamp silu(min(g, L)) * clamp(u, -L, L) at a limit that cuts a good share of the values."""
    k, n, K, cb = 256, 256, 3, 1
    tg, su, sg, tu, sv_u = _pair(k, n, K, seed=90 + m)
    x = make_x(m, k, seed=91)
    L = 1.5
    out = _run(x, tg, su, sg, tu, sv_u, K, cb, L)
    ref = _ref(x, tg, su, sg, tu, sv_u, K, cb, L)
    check_close(out.float().cpu().numpy(), ref, f"gate_up limit m={m}")


_CFG3 = {}


@pytest.mark.parametrize("M,rows_checked", [(16, 16), (2048, 64)])
def test_config3_gate_up_swiglu(M, rows_checked):
    """Config 3: in 4096, gate and up 14336 wide each, K=3 mul1, SiLU(gate)*up in fp16."""
    print(f"case: config 3 gate_up M={M}", flush=True)
    k, n, K, cb = 4096, 14336, 3, 2
    if not _CFG3:
        tg, su, sg, tu, sv_u = _pair(k, n, K, seed=33)
        _CFG3["w"] = (tg, su, sg, tu, sv_u)
        _CFG3["Wg"] = oracle.dequant(tg, su, sg, K, cb, rtz=True)
        _CFG3["Wu"] = oracle.dequant(tu, su, sv_u, K, cb, rtz=True)
    tg, su, sg, tu, sv_u = _CFG3["w"]
    x = make_x(M, k, seed=300 + M)
    out = _run(x, tg, su, sg, tu, sv_u, K, cb).float().cpu().numpy()
    rows = np.sort(np.random.default_rng(M).choice(M, size=rows_checked, replace=False))
    g = oracle.matmul(x[rows], _CFG3["Wg"])
    u = oracle.matmul(x[rows], _CFG3["Wu"])
    check_close(out[rows], oracle.swiglu(g, u, float("inf")), f"config 3 gate_up M={M}")


def test_gate_up_capi_rejects_bad_arguments():
    L = _lib.lib()
    assert L.exl3_gate_up_swiglu(None, None, None, None, None, None, None, 1, 256, 256, 3, 1, 0.0, None, 0,
                                 None) == _lib.EXL3_ERR_ARG
    assert b"null pointer" in L.exl3_last_error()
    assert L.exl3_gate_up_swiglu(1, 1, 1, 1, 1, 1, 1, 1, 250, 256, 3, 1, 0.0, None, 0, None) == _lib.EXL3_ERR_ARG
    assert L.exl3_gate_up_swiglu(4, 4, 16, 4, 16, 4, 4, 1, 256, 256, 3, 1, -1.0, None, 0, None) == _lib.EXL3_ERR_ARG
