"""GPU parity of the decode path: codebooks (exhaustive), tile layout, dequant (bit-exact).

The oracle (oracle/exl3_oracle.c) is pinned against the reference's own compiled
host header and the golden vectors in tests/test_oracle.py; here the HIP kernels
are compared with it bit for bit.
"""

import ctypes

import numpy as np
import pytest
import torch

import oracle
from gpu_util import make_weight, to_dev
from sglang_exl3 import _lib

pytestmark = pytest.mark.gpu


def _stream():
    return int(torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("cb", [0, 1, 2])
@pytest.mark.parametrize("rz", [True, False])
def test_codebook_table_exhaustive(cb, rz):
    print(f"case: codebook table cb={cb} rz={rz}", flush=True)
    states = torch.from_numpy(np.arange(65536, dtype=np.uint16).view(np.int16)).cuda()
    out = torch.empty(65536, dtype=torch.int16, device="cuda")
    rc = _lib.lib().exl3_decode_states(states.data_ptr(), 65536, cb, int(rz), out.data_ptr(), _stream())
    _lib.check(rc, "exl3_decode_states")
    got = out.cpu().numpy().view(np.uint16)
    want = oracle.codebook_table(cb, rz)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} mismatches, first state {bad[0]}: {got[bad[0]]:#06x} vs {want[bad[0]]:#06x}"


@pytest.mark.parametrize("K", [1, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("cb", [1, 2])
def test_decode_tiles_match_oracle(K, cb):
    print(f"case: decode_tiles K={K} cb={cb}", flush=True)
    k, n = 64, 96
    trellis, _, _ = make_weight(k, n, K, seed=100 + K)
    (tr,) = to_dev(trellis)
    W = torch.empty((k, n), dtype=torch.float16, device="cuda")
    rc = _lib.lib().exl3_decode_tiles(tr.data_ptr(), W.data_ptr(), k, n, K, cb, 1, _stream())
    _lib.check(rc, "exl3_decode_tiles")
    got = W.cpu().numpy().view(np.uint16)
    tu = trellis.view(np.uint16)
    for kt in range(k // 16):
        for nt in range(n // 16):
            want = oracle.decode_tile(tu[kt, nt], K, cb, rtz=True)
            blk = got[kt * 16:(kt + 1) * 16, nt * 16:(nt + 1) * 16]
            assert np.array_equal(blk, want), f"tile ({kt},{nt}) differs"


@pytest.mark.parametrize("K,cb,k,n", [(2, 1, 128, 256), (3, 2, 256, 128), (4, 1, 256, 384),
                                      (4, 2, 128, 128), (5, 1, 128, 256), (8, 2, 128, 128),
                                      (3, 0, 128, 256)])
def test_dequant_bit_exact(K, cb, k, n):
    print(f"case: dequant K={K} cb={cb} k={k} n={n}", flush=True)
    trellis, suh, svh = make_weight(k, n, K, seed=7 * K + cb)
    tr, su, sv = to_dev(trellis, suh, svh)
    W = torch.empty((k, n), dtype=torch.float16, device="cuda")
    rc = _lib.lib().exl3_dequant_trellis(tr.data_ptr(), su.data_ptr(), sv.data_ptr(), W.data_ptr(), k, n, K, cb,
                                         _stream())
    _lib.check(rc, "exl3_dequant_trellis")
    got = W.cpu().numpy().view(np.uint16)
    want = oracle.dequant(trellis, suh, svh, K, cb, rtz=True)
    bad = np.argwhere(got != want)
    assert bad.shape[0] == 0, f"{bad.shape[0]} differing fp16 words, first at {tuple(bad[0])}"


def test_dequant_torch_op_matches_oracle():
    from sglang_exl3 import ops

    ops.register_custom_ops()
    trellis, suh, svh = make_weight(256, 256, 4, seed=3)
    tr, su, sv = to_dev(trellis, suh, svh)
    W = torch.ops.sglang_exl3.dequant_trellis(tr, su, sv, 4, True)
    assert W.dtype == torch.float16 and tuple(W.shape) == (256, 256)
    want = oracle.dequant(trellis, suh, svh, 4, 1, rtz=True)
    assert np.array_equal(W.cpu().numpy().view(np.uint16), want)


def test_dequant_all_zero_trellis_closed_form():
    """Reference fixture (tests/test_cuda_graph.py:76-78) at a dequant-valid size: an all-zero
    trellis decodes every value to c = codebook(state 0), so per 128-block the two FWHT passes
    leave only the (0,0) corner, W = 128 * 128 * c * r^2 * suh * svh = 128 c suh svh, and every
    other entry is exactly 0.  c = 1.84375 (MCG), -3.453125 (mul1)."""
    from sglang_exl3 import ops

    ops.register_custom_ops()
    for mcg, c in ((True, 1.84375), (False, -3.453125)):
        k, n = 256, 256
        tr = torch.zeros((k // 16, n // 16, 32), dtype=torch.int16, device="cuda")
        su = torch.ones(k, dtype=torch.float16, device="cuda")
        sv = -torch.ones(n, dtype=torch.float16, device="cuda")
        Wn = torch.ops.sglang_exl3.dequant_trellis(tr, su, sv, 2, mcg).float().cpu().numpy()
        mask = np.ones_like(Wn, dtype=bool)
        mask[::128, ::128] = False
        assert np.all(Wn[mask] == 0.0)
        assert np.allclose(Wn[::128, ::128], -128.0 * c, rtol=1e-3)
