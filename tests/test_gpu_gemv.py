"""GPU parity of exl3_gemv / exl3_gemm / p2b_gemv_batched against the CPU oracle.

Bar: max-abs-err <= 2e-2 * rms(ref) and cosine >= 0.9999
against x @ dequant(W) accumulated in fp32 or better.  The dequantised W is the
oracle's (bit-exact restatement of the reference host dequant); at the full
full sizes the GPU dequant (pinned bit-exact in test_gpu_decode.py) stands in
for it, with a block spot-checked against the oracle.
"""

import numpy as np
import pytest
import torch

import oracle
from gpu_util import check_close, make_weight, make_x, to_dev
from sglang_exl3 import _lib, ops

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _registered():
    ops.register_custom_ops()


def _oracle_ref(x, trellis, suh, svh, K, cb):
    W = oracle.dequant(trellis, suh, svh, K, cb, rtz=True)
    return oracle.matmul(x, W)


@pytest.mark.parametrize("m,k,n,K,cb", [
    (1, 256, 256, 4, 1), (1, 512, 384, 3, 1), (2, 256, 512, 2, 1), (3, 384, 256, 4, 2),
    (8, 512, 256, 5, 1), (8, 256, 256, 3, 2), (4, 256, 256, 4, 0), (16, 256, 384, 4, 1),
    (17, 256, 256, 3, 1), (33, 256, 256, 4, 2), (64, 256, 256, 2, 1), (1, 256, 256, 1, 1),
    (2, 256, 256, 6, 2), (1, 256, 256, 7, 1), (5, 256, 256, 8, 1),
])
def test_gemv_small_vs_oracle(m, k, n, K, cb):
    print(f"case: gemv m={m} k={k} n={n} K={K} cb={cb}", flush=True)
    trellis, suh, svh = make_weight(k, n, K, seed=1000 + 17 * K + cb + m)
    x = make_x(m, k, seed=m * 31 + K)
    xd, tr, su, sv = to_dev(x, trellis, suh, svh)
    if cb == 0:
        y = _run_capi(xd, tr, su, sv, K, cb)
    else:
        y = torch.ops.sglang_exl3.exl3_gemv(xd, tr, su, sv, K, cb == 1, 1)
    torch.cuda.synchronize()
    assert y.shape == (m, n) and y.dtype == torch.float16
    ref = _oracle_ref(x, trellis, suh, svh, K, cb)
    check_close(y.float().cpu().numpy(), ref, f"gemv m={m} K={K} cb={cb}")


def _run_capi(xd, tr, su, sv, K, cb):
    m, k = xd.shape
    n = tr.shape[1] * 16
    y = torch.empty((m, n), dtype=torch.float16, device="cuda")
    L = _lib.lib()
    need = int(L.exl3_gemv_workspace_size(m, k, n, K, 1))
    ws = ops.workspace(xd.device, need) if need else None
    rc = L.exl3_gemv(xd.data_ptr(), tr.data_ptr(), su.data_ptr(), sv.data_ptr(), y.data_ptr(), m, k, n, K, cb,
                     0 if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(),
                     int(torch.cuda.current_stream().cuda_stream))
    _lib.check(rc, "exl3_gemv")
    return y


@pytest.mark.parametrize("m", [1, 2, 4, 8])
def test_gemv_baseline_config2_full_size(m):
    """Headline config 2: k=4096, n=14336, K=4, MCG, seeded random trellis, +-1 signs."""
    print(f"case: gemv cfg2 full size m={m}", flush=True)
    k, n, K = 4096, 14336, 4
    trellis, suh, svh = make_weight(k, n, K, seed=2)
    x = make_x(m, k, seed=20 + m)
    xd, tr, su, sv = to_dev(x, trellis, suh, svh)
    W = torch.ops.sglang_exl3.dequant_trellis(tr, su, sv, K, True)
    # spot-check one 128x128 block of the GPU dequant against the oracle
    blk = oracle.dequant(trellis[8:16, 40:48], suh[128:256], svh[640:768], K, 1, rtz=True)
    assert np.array_equal(W[128:256, 640:768].cpu().numpy().view(np.uint16), blk)
    ref = (xd.float() @ W.float()).cpu().numpy()
    y = torch.ops.sglang_exl3.exl3_gemv(xd, tr, su, sv, K, True, 1)
    check_close(y.float().cpu().numpy(), ref, f"cfg2 m={m}")


def test_gemv_deterministic():
    k, n, K = 2048, 4096, 3
    trellis, suh, svh = make_weight(k, n, K, seed=5)
    x = make_x(4, k, seed=5)
    xd, tr, su, sv = to_dev(x, trellis, suh, svh)
    y1 = torch.ops.sglang_exl3.exl3_gemv(xd, tr, su, sv, K, True, 1)
    y2 = torch.ops.sglang_exl3.exl3_gemv(xd, tr, su, sv, K, True, 1)
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))


def test_gemv_zero_trellis_closed_form():
    """All-zero trellis (the reference's own fixture, tests/test_cuda_graph.py:76-78): only
    output columns 128j are non-zero, y[:,128j] = 128 c svh[128j] sum_i x[:,128i] suh[128i]."""
    k, n = 512, 384
    for mcg, c in ((True, 1.84375), (False, -3.453125)):
        rng = np.random.default_rng(11)
        x = rng.standard_normal((2, k)).astype(np.float16)
        suh = np.where(rng.random(k) < 0.5, -1.0, 1.0).astype(np.float16)
        svh = np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float16)
        tr = torch.zeros((k // 16, n // 16, 32), dtype=torch.int16, device="cuda")
        xd, su, sv = to_dev(x, suh, svh)
        y = torch.ops.sglang_exl3.exl3_gemv(xd, tr, su, sv, 2, mcg, 1).float().cpu().numpy()
        s = (x.astype(np.float64)[:, ::128] * suh.astype(np.float64)[::128]).sum(axis=1)
        want = 128.0 * c * s[:, None] * svh.astype(np.float64)[None, ::128]
        assert np.allclose(y[:, ::128], want, rtol=2e-2, atol=1e-2 * np.abs(want).max())
        mask = np.ones(n, dtype=bool)
        mask[::128] = False
        assert np.abs(y[:, mask]).max() <= 1e-3 * np.abs(want).max()


@pytest.mark.parametrize("m,n", [(1, 256), (12, 256), (13, 256), (16, 256), (64, 256), (130, 256), (8, 12288),
                                 (9, 12288)])
def test_gemm_any_rows(m, n):
    """exl3_gemm on both sides of its GEMV / MFMA crossover (12 rows below
    12288 output columns, 8 from there)."""
    print(f"case: gemm m={m} n={n}", flush=True)
    k, K = 512, 3
    trellis, suh, svh = make_weight(k, n, K, seed=40 + m)
    x = make_x(m, k, seed=41 + m)
    xd, tr, su, sv = to_dev(x, trellis, suh, svh)
    y = torch.ops.sglang_exl3.exl3_gemm(xd, tr, su, sv, K, False)
    ref = _oracle_ref(x, trellis, suh, svh, K, 2)
    check_close(y.float().cpu().numpy(), ref, f"gemm m={m}")


@pytest.mark.parametrize("per_expert", [False, True])
def test_p2b_gemv_batched(per_expert):
    print(f"case: p2b_gemv_batched per_expert={per_expert}", flush=True)
    E, k, n, K, m = 6, 256, 384, 3, 2
    ws = [make_weight(k, n, K, seed=300 + e) for e in range(E)]
    dev = [to_dev(*w) for w in ws]
    tptr = torch.tensor([d[0].data_ptr() for d in dev], dtype=torch.int64, device="cuda")
    uptr = torch.tensor([d[1].data_ptr() for d in dev], dtype=torch.int64, device="cuda")
    vptr = torch.tensor([d[2].data_ptr() for d in dev], dtype=torch.int64, device="cuda")
    ids = [4, 0, 5, 4]
    idt = torch.tensor(ids, dtype=torch.int32, device="cuda")
    if per_expert:
        x = np.stack([make_x(m, k, seed=500 + j) for j in range(len(ids))])
    else:
        x = make_x(m, k, seed=500)
    (xd,) = to_dev(x)
    out = torch.ops.sglang_exl3.p2b_gemv_batched(xd, tptr, uptr, vptr, idt, K, True, n)
    assert out.shape == (len(ids), m, n)
    for j, e in enumerate(ids):
        xe = x[j] if per_expert else x
        ref = _oracle_ref(xe, *ws[e], K, 1)
        check_close(out[j].float().cpu().numpy(), ref, f"batched slot {j} expert {e}")


def test_gemv_rejects_bad_shapes():
    trellis, suh, svh = make_weight(256, 256, 4, seed=1)
    x = make_x(1, 256, seed=1)
    xd, tr, su, sv = to_dev(x, trellis, suh, svh)
    with pytest.raises(RuntimeError):
        torch.ops.sglang_exl3.exl3_gemv(xd, tr, su, sv, 3, True, 1)  # K does not match trellis
    with pytest.raises(RuntimeError):
        torch.ops.sglang_exl3.exl3_gemv(xd[:, :128].contiguous(), tr, su, sv, 4, True, 1)
    with pytest.raises(RuntimeError):
        torch.ops.sglang_exl3.exl3_gemv(xd.cpu(), tr, su, sv, 4, True, 1)


def _with_env(env, fn):
    import os
    old = {k: os.environ.get(k) for k in env}
    os.environ.update({k: str(v) for k, v in env.items()})
    try:
        return fn()
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


@pytest.mark.parametrize("k,n,K,cb,pieces", [
    # k/64 k-steps per column block in `pieces` equal pieces (1..16 steps each); every codebook,
    # up to 64 contributions per output (the fixed-point accumulators' limit is 63: 32 is the max here)
    (512, 384, 4, 1, 1), (512, 384, 4, 1, 2), (512, 384, 3, 2, 4), (512, 384, 2, 0, 8),
    (768, 256, 5, 2, 2), (768, 256, 4, 1, 3), (768, 256, 4, 0, 4), (1024, 256, 6, 1, 16),
    (2048, 128, 4, 1, 4), (640, 640, 4, 2, 10), (256, 256, 8, 0, 2), (4096, 256, 4, 1, 32),
    (1792, 512, 3, 1, 4), (4096, 384, 1, 2, 16), (3072, 256, 7, 1, 12),
])
def test_gemv_balanced_pieces(k, n, K, cb, pieces):
    """Balanced bs=1 kernel at forced piece counts over every instantiated piece length."""
    print(f"case: balanced gemv k={k} n={n} K={K} cb={cb} pieces={pieces}", flush=True)
    trellis, suh, svh = make_weight(k, n, K, seed=700 + pieces + 3 * K + cb)
    x = make_x(1, k, seed=701 + pieces)
    xd, tr, su, sv = to_dev(x, trellis, suh, svh)
    env = {"EXL3_GEMV_SK_P": pieces}
    plan = _with_env(env, lambda: _plan(1, k, n, K))
    assert plan[1] == (k // 64) // pieces and plan[2] == 1 and plan[3] == pieces
    ys = [_with_env(env, lambda: _run_capi(xd, tr, su, sv, K, cb)) for _ in range(2)]
    torch.cuda.synchronize()
    ref = _oracle_ref(x, trellis, suh, svh, K, cb)
    check_close(ys[0].float().cpu().numpy(), ref, f"balanced pieces={pieces}")
    # a second call on the same workspace gives the same bits (accumulators were cleared)
    assert torch.equal(ys[0].view(torch.int16), ys[1].view(torch.int16))


@pytest.mark.parametrize("m,k,n,K,cb,pieces", [
    (2, 512, 384, 4, 1, 2), (3, 768, 256, 3, 2, 3), (4, 1024, 256, 4, 0, 16), (4, 4096, 256, 2, 1, 8),
    (2, 2048, 128, 5, 2, 32), (3, 640, 640, 4, 1, 10),
])
def test_gemv_balanced_rows(m, k, n, K, cb, pieces):
    """Balanced kernel with 2..4 rows (A rows 0..m-1, one epilogue wave per row) at forced piece
    counts; a second call gives the same bits and the workspace zero regions are zero again."""
    print(f"case: balanced gemv rows m={m} k={k} n={n} K={K} cb={cb} pieces={pieces}", flush=True)
    trellis, suh, svh = make_weight(k, n, K, seed=750 + m + pieces + 3 * K + cb)
    x = make_x(m, k, seed=751 + m + pieces)
    xd, tr, su, sv = to_dev(x, trellis, suh, svh)
    env = {"EXL3_GEMV_SK_P": pieces, "EXL3_GEMV_SK_ROWS": 4}
    plan = _with_env(env, lambda: _plan(m, k, n, K))
    assert plan[1] == (k // 64) // pieces and plan[2] == 1 and plan[3] == pieces
    L = _lib.lib()
    need = int(L.exl3_gemv_workspace_size(m, k, n, K, 1))
    assert need >= 256 * 1024 + m * n * 8
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    ys = []
    for _ in range(2):
        y = torch.empty((m, n), dtype=torch.float16, device="cuda")
        rc = _with_env(env, lambda: L.exl3_gemv(xd.data_ptr(), tr.data_ptr(), su.data_ptr(), sv.data_ptr(),
                                                 y.data_ptr(), m, k, n, K, cb, ws.data_ptr(), ws.numel(),
                                                 int(torch.cuda.current_stream().cuda_stream)))
        _lib.check(rc, "exl3_gemv")
        torch.cuda.synchronize()
        assert int(torch.count_nonzero(ws)) == 0
        ys.append(y)
    check_close(ys[0].float().cpu().numpy(), _oracle_ref(x, trellis, suh, svh, K, cb), f"balanced rows m={m}")
    assert torch.equal(ys[0].view(torch.int16), ys[1].view(torch.int16))


def _plan(m, k, n, K):
    import ctypes
    out = (ctypes.c_int * 5)()
    _lib.check(_lib.lib().exl3_gemv_plan(m, k, n, K, 1, out), "exl3_gemv_plan")
    return list(out)


@pytest.mark.parametrize("m,k,n,K,cb", [(1, 512, 256, 4, 1), (8, 256, 384, 3, 2), (16, 512, 256, 2, 0)])
def test_gemv_split_kernel_vs_oracle(m, k, n, K, cb):
    """The k-split kernel (batched form, m > 16) on single-matrix problems too."""
    print(f"case: split gemv m={m} k={k} n={n} K={K} cb={cb}", flush=True)
    trellis, suh, svh = make_weight(k, n, K, seed=800 + m + K)
    x = make_x(m, k, seed=801 + m)
    xd, tr, su, sv = to_dev(x, trellis, suh, svh)
    assert _with_env({"EXL3_GEMV_SK": 0}, lambda: _plan(m, k, n, K))[2] >= 1
    y = _with_env({"EXL3_GEMV_SK": 0}, lambda: _run_capi(xd, tr, su, sv, K, cb))
    ref = _oracle_ref(x, trellis, suh, svh, K, cb)
    check_close(y.float().cpu().numpy(), ref, f"split m={m}")


@pytest.mark.parametrize("m,fx_rows", [(4, None), (8, None), (20, "32")])
def test_gemv_split_fixed_point_handoff(m, fx_rows):
    """k-split kernel whose splits add their rotated partial rows into the fixed-point
    accumulators (default up to 8 rows; 20 rows forced, two row blocks): against the
    oracle, bit-identical over repeated calls, the workspace zero again after each
    call, and close to the partial-tile hand-off (EXL3_GEMV_FX_ROWS=0)."""
    k, n, K, cb = 2048, 512, 3, 1
    print(f"case: split fixed-point gemv m={m} fx_rows={fx_rows}", flush=True)
    env = {"EXL3_GEMV_SK": 0} if fx_rows is None else {"EXL3_GEMV_SK": 0, "EXL3_GEMV_FX_ROWS": fx_rows}
    trellis, suh, svh = make_weight(k, n, K, seed=950 + m)
    x = make_x(m, k, seed=951 + m)
    xd, tr, su, sv = to_dev(x, trellis, suh, svh)
    assert _with_env(env, lambda: _plan(m, k, n, K))[3] > 1  # several k-splits
    L = _lib.lib()
    need = int(_with_env(env, lambda: L.exl3_gemv_workspace_size(m, k, n, K, 1)))
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    outs = []
    for _ in range(3):
        y = torch.empty((m, n), dtype=torch.float16, device="cuda")
        _with_env(env, lambda: _lib.check(
            L.exl3_gemv(xd.data_ptr(), tr.data_ptr(), su.data_ptr(), sv.data_ptr(), y.data_ptr(), m, k, n, K, cb,
                        ws.data_ptr(), ws.numel(), int(torch.cuda.current_stream().cuda_stream)), "exl3_gemv"))
        torch.cuda.synchronize()
        assert int(torch.count_nonzero(ws)) == 0
        outs.append(y)
    for y in outs[1:]:
        assert torch.equal(y, outs[0]), "fixed-point hand-off: repeated calls differ"
    check_close(outs[0].float().cpu().numpy(), _oracle_ref(x, trellis, suh, svh, K, cb), f"fx m={m}")
    tiles = _with_env({"EXL3_GEMV_SK": 0, "EXL3_GEMV_FX_ROWS": "0"}, lambda: _run_capi(xd, tr, su, sv, K, cb))
    check_close(outs[0].float().cpu().numpy(), tiles.float().cpu().numpy(), f"fx vs tiles m={m}")


def test_gemv_balanced_leaves_accumulators_zero():
    """Every output element's fixed-point accumulator is cleared by the workgroup that
    completes it, so the workspace's zero regions are zero after each call."""
    m, k, n, K = 1, 1024, 2048, 4
    assert _plan(m, k, n, K)[2] == 1  # the balanced kernel serves m <= 2
    trellis, suh, svh = make_weight(k, n, K, seed=900)
    x = make_x(m, k, seed=901)
    xd, tr, su, sv = to_dev(x, trellis, suh, svh)
    L = _lib.lib()
    need = int(L.exl3_gemv_workspace_size(m, k, n, K, 1))
    assert need >= 256 * 1024 + m * n * 8
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    y = torch.empty((m, n), dtype=torch.float16, device="cuda")
    for _ in range(3):
        _lib.check(L.exl3_gemv(xd.data_ptr(), tr.data_ptr(), su.data_ptr(), sv.data_ptr(), y.data_ptr(), m, k, n, K,
                               1, ws.data_ptr(), ws.numel(), int(torch.cuda.current_stream().cuda_stream)),
                   "exl3_gemv")
        torch.cuda.synchronize()
        assert int(torch.count_nonzero(ws)) == 0
    check_close(y.float().cpu().numpy(), _oracle_ref(x, trellis, suh, svh, K, 1), "balanced ws")


def test_workspace_growth_keeps_captured_graphs_valid():
    """A graph captured with the stream's workspace stays correct after a larger
    op grew that workspace (the old buffer is kept alive, not freed); growth
    itself is refused during capture."""
    k, n, K = 512, 1024, 4
    tr, su, sv = make_weight(k, n, K, seed=71)
    x = make_x(8, k, seed=72)
    d = to_dev(x, tr, su, sv)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        torch.ops.sglang_exl3.exl3_gemv(*d, K, True, 1)  # sizes the stream's workspace
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            y = torch.ops.sglang_exl3.exl3_gemv(*d, K, True, 1)
        # grow the workspace of the same stream well past its first size
        kb, nb = 4096, 8192
        trb, sub, svb = make_weight(kb, nb, 2, seed=73)
        xb = make_x(64, kb, seed=74)
        yb = torch.ops.sglang_exl3.exl3_gemv(*to_dev(xb, trb, sub, svb), 2, True, 1)
        for _ in range(3):
            g.replay()
    torch.cuda.synchronize()
    ref = oracle.matmul(x, oracle.dequant(tr, su, sv, K, 1, rtz=True))
    check_close(y.float().cpu().numpy(), ref, "graph replay after workspace growth")
    assert yb.shape == (64, nb)
    # an op whose workspace would have to grow during capture is refused with a clear message
    s2 = torch.cuda.Stream()
    g2 = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="during HIP graph capture"):
        with torch.cuda.stream(s2):
            with torch.cuda.graph(g2, stream=s2):
                torch.ops.sglang_exl3.exl3_gemv(*d, K, True, 1)
