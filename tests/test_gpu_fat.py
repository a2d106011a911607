"""GPU parity of the many-row MFMA GEMM: exl3_fat_gemm / exl3_fat_gemm_scatter
(rotated fp16 input, fp32 output) and exl3_gemm's prefill path (m ≥ 12),
against the oracle (bar: max-abs-err <= 2e-2 * rms(ref), cosine >= 0.9999)."""

import numpy as np
import pytest
import torch

import oracle
from gpu_util import check_close, make_weight, make_x
from sglang_exl3 import ops

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _registered():
    ops.register_custom_ops()


def _rotate(x, suh):
    """fp16(H(x * suh) / sqrt(128)) per 128 block (the input the fat GEMM takes)."""
    return oracle.had_rows(x.astype(np.float32), suh, None, np.float32(0.08838834764831845)).astype(np.float16)


def _ref(a_rot, trellis, svh, K, cb):
    """svh * H(a_rot . T) / sqrt(128), with T the decoded tiles (no rotations)."""
    k, n = trellis.shape[0] * 16, trellis.shape[1] * 16
    ones_k = np.ones(k, dtype=np.float16)
    ones_n = np.ones(n, dtype=np.float16)
    # the oracle's dequant W = suh*svh*(H T H)/128; with unit scales, H W H = 128 T... use decode_tile directly
    T = np.zeros((k, n), dtype=np.float32)
    for kt in range(k // 16):
        for nt in range(n // 16):
            T[kt * 16:(kt + 1) * 16, nt * 16:(nt + 1) * 16] = oracle.f16_to_f32(
                oracle.decode_tile(trellis[kt, nt].view(np.uint16), K, cb, rtz=False))
    y = a_rot.astype(np.float64) @ T.astype(np.float64)
    del ones_k, ones_n
    return oracle.had_rows(y.astype(np.float32), None, svh, np.float32(0.08838834764831845))


@pytest.mark.parametrize("M,k,n,K,cb", [
    (16, 256, 256, 4, 1), (1, 256, 128, 3, 2), (40, 512, 384, 3, 1), (128, 256, 256, 4, 0),
    (200, 1024, 256, 2, 2), (300, 256, 512, 5, 1),
])
def test_fat_gemm_vs_oracle(M, k, n, K, cb):
    print(f"case: fat M={M} k={k} n={n} K={K} cb={cb}", flush=True)
    tr, su, sv = make_weight(k, n, K, seed=M * 13 + K)
    x = make_x(M, k, seed=M)
    a = _rotate(x, su)
    out = torch.full((M, n), 123.0, dtype=torch.float32, device="cuda")  # overwritten
    mcg, mul1 = cb == 1, cb == 2
    torch.ops.sglang_exl3.exl3_fat_gemm(torch.from_numpy(a).cuda(), torch.from_numpy(tr).cuda(), out,
                                        torch.from_numpy(sv).cuda(), K, mcg, mul1)
    torch.cuda.synchronize()
    check_close(out.cpu().numpy(), _ref(a, tr, sv, K, cb), f"fat M={M}")


def _with_env(name, value, fn):
    import os
    old = os.environ.get(name)
    os.environ[name] = value
    try:
        return fn()
    finally:
        if old is None:
            del os.environ[name]
        else:
            os.environ[name] = old


def _fat(a, tr, sv, K, cb, M, n):
    out = torch.full((M, n), 123.0, dtype=torch.float32, device="cuda")  # overwritten
    torch.ops.sglang_exl3.exl3_fat_gemm(torch.from_numpy(a).cuda(), torch.from_numpy(tr).cuda(), out,
                                        torch.from_numpy(sv).cuda(), K, cb == 1, cb == 2)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("K", range(1, 9))
@pytest.mark.parametrize("cb", [0, 1, 2])
def test_fat_wide_tiles_every_width(K, cb):
    """Wide-tile kernel (256 x 256 tiles, above 256 rows): every bit width and codebook,
    a partial second row tile (ending in the first row half), k-splits accumulating atomically."""
    M, k, n = 300, 256, 256
    print(f"case: fat wide M={M} k={k} n={n} K={K} cb={cb}", flush=True)
    tr, su, sv = make_weight(k, n, K, seed=100 + 3 * K + cb)
    a = _rotate(make_x(M, k, seed=K + 10 * cb), su)
    out = _with_env("EXL3_FAT_WIDE", "2", lambda: _fat(a, tr, sv, K, cb, M, n))
    check_close(out, _ref(a, tr, sv, K, cb), f"fat wide K={K} cb={cb}")


@pytest.mark.parametrize("M,k,n,K,cb", [(512, 1024, 512, 3, 2), (257, 512, 768, 4, 1), (65, 2048, 256, 2, 0),
                                        (1100, 128, 512, 5, 1)])
@pytest.mark.parametrize("wide", ["2", "1", "0"])
def test_fat_wide_and_narrow_kernels(M, k, n, K, cb, wide):
    """The same shapes through the wide-tile kernel (EXL3_FAT_WIDE=2), the
    default plan and the narrow kernel (EXL3_FAT_WIDE=0)."""
    print(f"case: fat M={M} k={k} n={n} K={K} cb={cb} wide={wide}", flush=True)
    tr, su, sv = make_weight(k, n, K, seed=M + n)
    a = _rotate(make_x(M, k, seed=M + 1), su)
    out = _with_env("EXL3_FAT_WIDE", wide, lambda: _fat(a, tr, sv, K, cb, M, n))
    check_close(out, _ref(a, tr, sv, K, cb), f"fat M={M} wide={wide}")


def test_fat_wide_scatter_accumulates(monkeypatch):
    monkeypatch.setenv("EXL3_FAT_WIDE", "2")  # the wide-tile kernel at this small grid
    M, k, n, K = 300, 512, 512, 3
    tr, su, sv = make_weight(k, n, K, seed=15)
    a = _rotate(make_x(M, k, seed=16), su)
    rng = np.random.default_rng(17)
    tok = rng.integers(0, 40, size=M).astype(np.int64)
    rw = (rng.random(M) + 0.5).astype(np.float16)
    base = rng.standard_normal((40, n)).astype(np.float32)
    out = torch.from_numpy(base.copy()).cuda()
    torch.ops.sglang_exl3.exl3_fat_gemm_scatter(torch.from_numpy(a).cuda(), torch.from_numpy(tr).cuda(), out,
                                                torch.from_numpy(sv).cuda(), torch.from_numpy(tok).cuda(),
                                                torch.from_numpy(rw).cuda(), K, False, True)
    torch.cuda.synchronize()
    rows = _ref(a, tr, sv, K, 2) * rw.astype(np.float32)[:, None]
    want = base.copy()
    np.add.at(want, tok, rows)
    check_close(out.cpu().numpy() - base, want - base, "fat wide scatter")


def test_fat_gemm_scatter_accumulates():
    M, k, n, K = 48, 256, 256, 4
    tr, su, sv = make_weight(k, n, K, seed=5)
    x = make_x(M, k, seed=6)
    a = _rotate(x, su)
    rng = np.random.default_rng(7)
    tok = rng.integers(0, 20, size=M).astype(np.int64)  # destinations repeat: atomics
    rw = (rng.random(M) + 0.5).astype(np.float16)
    base = rng.standard_normal((20, n)).astype(np.float32)
    out = torch.from_numpy(base.copy()).cuda()
    torch.ops.sglang_exl3.exl3_fat_gemm_scatter(torch.from_numpy(a).cuda(), torch.from_numpy(tr).cuda(), out,
                                                torch.from_numpy(sv).cuda(), torch.from_numpy(tok).cuda(),
                                                torch.from_numpy(rw).cuda(), K, True, False)
    torch.cuda.synchronize()
    rows = _ref(a, tr, sv, K, 1) * rw.astype(np.float32)[:, None]
    want = base.copy()
    np.add.at(want, tok, rows)
    check_close(out.cpu().numpy() - base, want - base, "fat scatter")


@pytest.mark.parametrize("m,k,n,K,cb", [(65, 256, 256, 4, 1), (200, 512, 384, 3, 2), (1000, 256, 128, 2, 1),
                                        (300, 128, 512, 3, 1), (700, 1024, 256, 4, 2)])
def test_gemm_prefill_path_vs_oracle(m, k, n, K, cb):
    print(f"case: gemm prefill m={m} k={k} n={n}", flush=True)
    tr, su, sv = make_weight(k, n, K, seed=m + k)
    x = make_x(m, k, seed=m)
    y = torch.ops.sglang_exl3.exl3_gemm(torch.from_numpy(x).cuda(), torch.from_numpy(tr).cuda(),
                                        torch.from_numpy(su).cuda(), torch.from_numpy(sv).cuda(), K, cb == 1)
    torch.cuda.synchronize()
    ref = oracle.matmul(x, oracle.dequant(tr, su, sv, K, cb, rtz=True))
    check_close(y.float().cpu().numpy(), ref, f"gemm prefill m={m}")


def test_fat_then_gemv_workspace_stays_clean():
    """The prefill scratch must not disturb the GEMV counters sharing the workspace."""
    k, n, K = 512, 1024, 4
    tr, su, sv = make_weight(k, n, K, seed=1)
    d = [torch.from_numpy(v).cuda() for v in (tr, su, sv)]
    xb = make_x(300, k, seed=2)
    torch.ops.sglang_exl3.exl3_gemm(torch.from_numpy(xb).cuda(), *d, K, True)
    xs = make_x(2, k, seed=3)
    y = torch.ops.sglang_exl3.exl3_gemv(torch.from_numpy(xs).cuda(), *d, K, True, 1)
    torch.cuda.synchronize()
    check_close(y.float().cpu().numpy(), oracle.matmul(xs, oracle.dequant(tr, su, sv, K, 1, rtz=True)), "gemv after")


@pytest.mark.parametrize("cb", [1, 2])
@pytest.mark.parametrize("op", ["gemm", "gate_up"])
def test_tail_split_repeatable(op, cb, monkeypatch):
    """Tail split of the wide-tile kernel (every tile of a one-round launch runs as
    two k-halves, the first half hands its sums to the second): against the
    oracle, bit-identical over repeated calls (the hand-off counts and flags
    reset themselves), and close to the unsplit kernel (EXL3_FAT_TAIL=0)."""
    # gemm: 56 x 2 tiles, enough for one k-split (smaller grids split k with
    # fp32 atomics instead); gate/up: 2 x 2 tiles, always one split
    m, k, K = (512, 1024, 3) if op == "gemm" else (300, 1024, 3)
    n = 14336 if op == "gemm" else 256
    print(f"case: tail split {op} m={m} k={k} n={n} cb={cb}", flush=True)
    x = torch.from_numpy(make_x(m, k, seed=31)).cuda()
    if op == "gemm":
        tr, su, sv = make_weight(k, n, K, seed=32)
        d = [torch.from_numpy(v).cuda() for v in (tr, su, sv)]
        run = lambda: torch.ops.sglang_exl3.exl3_gemm(x, *d, K, cb == 1)
        ref = oracle.matmul(x.cpu().numpy(), oracle.dequant(tr, su, sv, K, cb, rtz=True))
    else:
        tg, su, sg = make_weight(k, n, K, seed=33)
        tu, _, su2 = make_weight(k, n, K, seed=34)
        d = [torch.from_numpy(v).cuda() for v in (su, tg, sg, tu, su2)]
        run = lambda: torch.ops.sglang_exl3.exl3_gate_up_swiglu(x, *d, K, cb)
        g = oracle.matmul(x.cpu().numpy(), oracle.dequant(tg, su, sg, K, cb, rtz=True))
        u = oracle.matmul(x.cpu().numpy(), oracle.dequant(tu, su, su2, K, cb, rtz=True))
        ref = oracle.swiglu(g, u, float("inf"))
    outs = [run() for _ in range(3)]
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o, outs[0]), "tail split: repeated calls differ"
    check_close(outs[0].float().cpu().numpy(), ref, f"tail split {op}")
    monkeypatch.setenv("EXL3_FAT_TAIL", "0")
    whole = run()
    torch.cuda.synchronize()
    check_close(outs[0].float().cpu().numpy(), whole.float().cpu().numpy(), f"tail split vs whole {op}")


@pytest.mark.parametrize("op,m", [("gemm", 16), ("gemm", 48), ("gemm", 300), ("gate_up", 16), ("gate_up", 48),
                                  ("gate_up", 200)])
def test_mul1_raw_entries(op, m, monkeypatch):
    """Narrow 16-row MFMA tiles on mul1 weights read raw entries (1024 + byte
    sum, no affine step) and correct in the epilogue with kinv * acc + bias *
    (row sum of the rotated x over the split's k range).  k = 14336 (112 chunk
    sums per row), 16-row tiles with k-splits (m = 16): against the oracle and
    close to the decoded path (EXL3_FAT_RAW=0).  The wide tiles in gate/up mode
    (m = 200: tail-split k-halves, the row sums taken in the epilogue) read
    raw entries too; the 64-row tiles (m = 48) and the plain wide tiles (gemm
    m = 300, forced by EXL3_FAT_WIDE=2: 16 fp32-atomic k-splits) decode values
    and are checked at the same k."""
    k, n, K, cb = 14336, 256, 3, 2
    if op == "gemm" and m > 256:
        monkeypatch.setenv("EXL3_FAT_WIDE", "2")
    print(f"case: raw mul1 {op} m={m} k={k} n={n}", flush=True)
    x = torch.from_numpy(make_x(m, k, seed=51 + m)).cuda()
    if op == "gemm":
        tr, su, sv = make_weight(k, n, K, seed=52)
        d = [torch.from_numpy(v).cuda() for v in (tr, su, sv)]
        run = lambda: torch.ops.sglang_exl3.exl3_gemm(x, *d, K, False)
        ref = oracle.matmul(x.cpu().numpy(), oracle.dequant(tr, su, sv, K, cb, rtz=True))
    else:
        tg, su, sg = make_weight(k, n, K, seed=53)
        tu, _, su2 = make_weight(k, n, K, seed=54)
        # svh / 16 keeps silu(g) * u inside fp16 at this k
        sg, su2 = (sg / 16).astype(np.float16), (su2 / 16).astype(np.float16)
        d = [torch.from_numpy(v).cuda() for v in (su, tg, sg, tu, su2)]
        run = lambda: torch.ops.sglang_exl3.exl3_gate_up_swiglu(x, *d, K, cb)
        g = oracle.matmul(x.cpu().numpy(), oracle.dequant(tg, su, sg, K, cb, rtz=True))
        u = oracle.matmul(x.cpu().numpy(), oracle.dequant(tu, su, su2, K, cb, rtz=True))
        ref = oracle.swiglu(g, u, float("inf"))
    raw = run()
    torch.cuda.synchronize()
    check_close(raw.float().cpu().numpy(), ref, f"raw mul1 {op} m={m}")
    monkeypatch.setenv("EXL3_FAT_RAW", "0")
    dec = run()
    torch.cuda.synchronize()
    check_close(raw.float().cpu().numpy(), dec.float().cpu().numpy(), f"raw vs decoded {op} m={m}")


@pytest.mark.parametrize("m,cb", [(16, 1), (64, 2)])
def test_gemm_split_handoff_repeatable(m, cb, monkeypatch):
    """exl3_gemm's narrow k-splits hand partial tiles to the last split of each
    (column block, row tile): against the oracle, bit-identical over repeated
    calls (the counters reset themselves), and close to the fp32-atomic path
    (EXL3_FAT_HANDOFF=0).  k = 4096, n = 2048: four splits of 16 steps."""
    k, n, K = 4096, 2048, 3
    print(f"case: gemm split hand-off m={m} cb={cb}", flush=True)
    x = torch.from_numpy(make_x(m, k, seed=61 + m)).cuda()
    tr, su, sv = make_weight(k, n, K, seed=62)
    d = [torch.from_numpy(v).cuda() for v in (tr, su, sv)]
    run = lambda: torch.ops.sglang_exl3.exl3_gemm(x, *d, K, cb == 1)
    outs = [run() for _ in range(3)]
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o, outs[0]), "split hand-off: repeated calls differ"
    ref = oracle.matmul(x.cpu().numpy(), oracle.dequant(tr, su, sv, K, cb, rtz=True))
    check_close(outs[0].float().cpu().numpy(), ref, f"split hand-off m={m}")
    monkeypatch.setenv("EXL3_FAT_HANDOFF", "0")
    atomic = run()
    torch.cuda.synchronize()
    check_close(outs[0].float().cpu().numpy(), atomic.float().cpu().numpy(), f"hand-off vs atomics m={m}")


@pytest.mark.parametrize("m,cb", [(6, 2), (9, 1), (13, 0), (16, 2)])
def test_gemm_split_out_finish_matches_in_kernel_handoff(m, cb, monkeypatch):
    """From 6 to 16 rows exl3_gemm's narrow k-splits store their partial tiles
    and a second launch (fat_split_finish_kernel) finishes every row; its sums
    and epilogue are the in-kernel hand-off's, so both give the same bits
    (EXL3_FAT_SPLIT_OUT=0 keeps the hand-off), mul1 raw entries included."""
    k, n, K = 2048, 384, 3
    print(f"case: gemm split-out finish m={m} cb={cb}", flush=True)
    monkeypatch.setenv("EXL3_GEMM_GEMV_ROWS", "0")  # the MFMA path at every m
    x = torch.from_numpy(make_x(m, k, seed=81 + m)).cuda()
    tr, su, sv = make_weight(k, n, K, seed=82 + cb)
    d = [torch.from_numpy(v).cuda() for v in (tr, su, sv)]
    run = lambda: torch.ops.sglang_exl3.exl3_linear(x, *d, K, cb)
    split = run()
    monkeypatch.setenv("EXL3_FAT_SPLIT_OUT", "0")
    handoff = run()
    torch.cuda.synchronize()
    assert torch.equal(split.view(torch.int16), handoff.view(torch.int16))
    ref = oracle.matmul(x.cpu().numpy(), oracle.dequant(tr, su, sv, K, cb, rtz=True))
    check_close(split.float().cpu().numpy(), ref, f"split-out m={m} cb={cb}")


@pytest.mark.parametrize("m", [13, 40, 100, 250])
@pytest.mark.parametrize("cb", [0, 1, 2])
def test_gemm_split_handoff_ragged_rows(m, cb):
    """The split hand-off on row counts that leave the last row tile partial
    (16-row tiles at 13 rows, 64-row tiles above), every codebook (3INST
    through exl3_linear): k = 2048 gives two splits of 16 steps, n = 384 three
    column blocks.  Against the oracle, and bit-identical on a repeat call."""
    k, n, K = 2048, 384, 4
    print(f"case: gemm split hand-off ragged m={m} cb={cb}", flush=True)
    x = torch.from_numpy(make_x(m, k, seed=71 + m)).cuda()
    tr, su, sv = make_weight(k, n, K, seed=72 + cb)
    d = [torch.from_numpy(v).cuda() for v in (tr, su, sv)]
    run = lambda: torch.ops.sglang_exl3.exl3_linear(x, *d, K, cb)
    first, again = run(), run()
    torch.cuda.synchronize()
    assert torch.equal(first, again), "split hand-off: repeated calls differ"
    ref = oracle.matmul(x.cpu().numpy(), oracle.dequant(tr, su, sv, K, cb, rtz=True))
    check_close(first.float().cpu().numpy(), ref, f"split hand-off ragged m={m} cb={cb}")


@pytest.mark.parametrize("K", range(1, 9))
@pytest.mark.parametrize("cb", [0, 1, 2])
def test_fat_narrow_every_width(K, cb):
    """Narrow kernel (64-row tiles, fp32 output through exl3_fat_gemm) at every
    bit width and codebook: the decode's windows (middle words for the ones
    that straddle two words) differ per K."""
    M, k, n = 24, 512, 256
    print(f"case: fat narrow M={M} k={k} n={n} K={K} cb={cb}", flush=True)
    tr, su, sv = make_weight(k, n, K, seed=200 + 3 * K + cb)
    a = _rotate(make_x(M, k, seed=K + 20 * cb), su)
    check_close(_fat(a, tr, sv, K, cb, M, n), _ref(a, tr, sv, K, cb), f"fat narrow K={K} cb={cb}")


@pytest.mark.parametrize("K", range(1, 9))
@pytest.mark.parametrize("cb", [1, 2])
def test_gemm_16_rows_every_width(K, cb):
    """exl3_gemm at 16 rows (16-row tiles, k-split hand-off; mul1 reads raw
    entries) at every bit width, against the oracle."""
    m, k, n = 16, 1024, 256
    print(f"case: gemm 16 rows K={K} cb={cb}", flush=True)
    tr, su, sv = make_weight(k, n, K, seed=300 + 3 * K + cb)
    x = make_x(m, k, seed=301 + K)
    d = [torch.from_numpy(v).cuda() for v in (x, tr, su, sv)]
    y = torch.ops.sglang_exl3.exl3_gemm(*d, K, cb == 1)
    torch.cuda.synchronize()
    ref = oracle.matmul(x, oracle.dequant(tr, su, sv, K, cb, rtz=True))
    check_close(y.float().cpu().numpy(), ref, f"gemm 16 rows K={K} cb={cb}")
