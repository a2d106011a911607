"""exl3_gemv_noalloc (the allocation-free variant of exl3_gemv) against
exl3_gemv with a caller workspace, through the C ABI: two calls in a row, the
second with a smaller input, each bit-identical to exl3_gemv (the same kernels
and launch plan) and within the matmul tolerance of the oracle."""

import numpy as np
import pytest
import torch

import oracle
from gpu_util import check_close, make_weight, make_x, to_dev
from sglang_exl3 import _lib

pytestmark = pytest.mark.gpu


def _gemv_ws(L, xd, tr, su, sv, m, k, n, K, cb, stream):
    y = torch.empty((m, n), dtype=torch.float16, device="cuda")
    need = int(L.exl3_gemv_workspace_size(m, k, n, K, 1))
    ws = torch.zeros(max(need, 256), dtype=torch.uint8, device="cuda")
    rc = L.exl3_gemv(xd.data_ptr(), tr.data_ptr(), su.data_ptr(), sv.data_ptr(), y.data_ptr(), m, k, n, K, cb,
                     ws.data_ptr(), ws.numel(), stream)
    _lib.check(rc, "exl3_gemv")
    return y


def _gemv_noalloc(L, xd, tr, su, sv, m, k, n, K, cb, stream):
    y = torch.empty((m, n), dtype=torch.float16, device="cuda")
    rc = L.exl3_gemv_noalloc(xd.data_ptr(), tr.data_ptr(), su.data_ptr(), sv.data_ptr(), y.data_ptr(), m, k, n, K,
                             cb, stream)
    _lib.check(rc, "exl3_gemv_noalloc")
    return y


# (m, k, n, K, codebook): the first shape takes the k-split kernel (partials and
# counters in the scratch), the second the balanced one (fixed-point accumulators)
@pytest.mark.parametrize("first,second", [
    ((8, 2048, 1024, 4, 1), (1, 512, 256, 3, 2)),
    ((2, 1024, 768, 2, 0), (1, 256, 128, 4, 1)),
])
def test_gemv_noalloc_matches_gemv(first, second):
    L = _lib.lib()
    stream = int(torch.cuda.current_stream().cuda_stream)
    for seed, (m, k, n, K, cb) in enumerate((first, second)):
        print(f"noalloc case m={m} k={k} n={n} K={K} cb={cb}", flush=True)
        trellis, suh, svh = make_weight(k, n, K, seed=40 + seed)
        x = make_x(m, k, seed=41 + seed)
        xd, tr, su, sv = to_dev(x, trellis, suh, svh)
        y_ref = _gemv_ws(L, xd, tr, su, sv, m, k, n, K, cb, stream)
        y = _gemv_noalloc(L, xd, tr, su, sv, m, k, n, K, cb, stream)
        y2 = _gemv_noalloc(L, xd, tr, su, sv, m, k, n, K, cb, stream)  # scratch left clean by the first call
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16)), "noalloc differs from exl3_gemv"
        assert torch.equal(y2.view(torch.int16), y_ref.view(torch.int16)), "second noalloc call differs"
        W = oracle.dequant(trellis, suh, svh, K, cb, rtz=True)
        check_close(y.float().cpu().numpy(), oracle.matmul(x, W), f"noalloc m={m} k={k} n={n}")
