"""GPU parity of the row Hadamard transform (exl3_hadamard_rows) against the
oracle: bit-exact fp16 (same fp32 operations in the same order, one final
rounding), including the DPP / permlane lane exchanges of every FWHT stage."""

import numpy as np
import pytest
import torch

import oracle
from sglang_exl3 import _lib
from sglang_exl3.hadamard_cache import HAD_NORM, hadamard_rows, transform_hadamard_fast

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,cols,use_pre,use_post,scale", [
    (1, 128, False, False, 1.0), (3, 256, True, False, HAD_NORM), (5, 512, False, True, HAD_NORM),
    (7, 1024, True, True, 0.5), (64, 4096, True, True, HAD_NORM), (1000, 128, True, False, 2.0),
])
def test_hadamard_rows_bit_exact(rows, cols, use_pre, use_post, scale):
    print(f"case: hadamard rows={rows} cols={cols} pre={use_pre} post={use_post}", flush=True)
    rng = np.random.default_rng(rows * 7 + cols)
    x = rng.standard_normal((rows, cols)).astype(np.float16)
    pre = rng.choice([-1.0, 1.0, 0.5], cols).astype(np.float16) if use_pre else None
    post = rng.choice([-1.0, 1.0, 0.25], cols).astype(np.float16) if use_post else None
    dev = lambda a: None if a is None else torch.from_numpy(a).cuda()
    y = hadamard_rows(dev(x), dev(pre), dev(post), scale)
    torch.cuda.synchronize()
    want = oracle.had_rows(x.astype(np.float32), pre, post, np.float32(scale)).astype(np.float16)
    assert np.array_equal(y.cpu().numpy().view(np.uint16), want.view(np.uint16))


def test_hadamard_rows_in_place_and_lane_layout():
    """A one-hot input in each lane position: exercises every lane exchange; y aliases x."""
    x = torch.zeros((128, 128), dtype=torch.float16, device="cuda")
    x[torch.arange(128), torch.arange(128)] = 1.0
    hadamard_rows(x, None, None, 1.0, out=x)
    H = np.array([[1.0]])
    while H.shape[0] < 128:
        H = np.block([[H, H], [H, -H]])
    assert np.array_equal(x.float().cpu().numpy(), H)


def test_transform_hadamard_fast_involution_and_suh():
    x = torch.randn((2, 256), dtype=torch.float32, device="cuda")
    h1 = transform_hadamard_fast(x)
    assert h1.shape == x.shape and h1.dtype == x.dtype
    torch.testing.assert_close(transform_hadamard_fast(h1), x, rtol=1e-2, atol=1e-2)
    suh = torch.where(torch.rand(256, device="cuda") < 0.5, -1.0, 1.0).half()
    h2 = transform_hadamard_fast(x, suh)
    torch.testing.assert_close(h2, h1 * suh.float(), rtol=0, atol=0)
    odd = torch.randn((2, 100), device="cuda")
    assert transform_hadamard_fast(odd) is odd


def test_hadamard_rejects_bad_shapes():
    L = _lib.lib()
    assert L.exl3_hadamard_rows(None, None, None, None, 1.0, 1, 100, None) == _lib.EXL3_ERR_ARG
    with pytest.raises(RuntimeError, match="multiple of 128"):
        hadamard_rows(torch.zeros((1, 100), dtype=torch.float16, device="cuda"))
