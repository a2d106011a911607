"""GPU parity of the row Hadamard transforms against the oracle:
exl3_hadamard_rows bit-exact in fp16 (same fp32 operations in the same order,
one final rounding), including the DPP / permlane lane exchanges of every FWHT
stage; exl3_hadamard_fast (transform_hadamard_fast) in fp16, bf16 and fp32
with the reference's scale and roundings."""

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


_TDT = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("rows,cols,post_kind", [(1, 128, None), (5, 512, "sign"), (33, 4096, "mixed"),
                                                 (1000, 256, "sign"), (2, 384, "mixed")])
def test_transform_hadamard_fast_matches_oracle(dtype, rows, cols, post_kind):
    """exl3_hadamard_fast against oracle.had_fast (exact block sum, the
    reference's dtype-rounded scale and its two roundings).  Only the fp32
    block sum's order differs (FWHT stages here, a matmul in the reference),
    so fp16 / bf16 results are bit-identical except where the exact value lies
    within a few fp32 ulps of a rounding boundary (then one ulp apart, for at
    most 2e-3 of the elements), and fp32 results lie within the FWHT's
    rounding bound, 8 ulps of sum |x| h."""
    print(f"case: hadamard_fast dtype={dtype} rows={rows} cols={cols} post={post_kind}", flush=True)
    rng = np.random.default_rng(rows * 13 + cols + len(dtype))
    x = oracle.round_to(rng.standard_normal((rows, cols)).astype(np.float32) * 3.0, dtype)
    post = None
    if post_kind == "sign":
        post = rng.choice([-1.0, 1.0], cols).astype(np.float32)
    elif post_kind == "mixed":
        post = rng.choice([-1.0, 1.0, 0.5, -2.0, 1.5, 0.7], cols).astype(np.float32)
    xt = torch.from_numpy(x).to(_TDT[dtype]).cuda()
    suh = None if post is None else torch.from_numpy(post).half().cuda()
    y = transform_hadamard_fast(xt, suh)
    torch.cuda.synchronize()
    assert y.dtype == xt.dtype and y.shape == xt.shape
    got = y.float().cpu().numpy()
    want = oracle.had_fast(x, None if post is None else post.astype(np.float16), dtype)
    if dtype == "f32":
        h = float(np.float32(0.08838834764831845))
        mag = np.repeat(np.abs(x).reshape(rows, cols // 128, 128).sum(-1), 128, axis=1) * h
        if post is not None:
            mag = mag * np.abs(post)[None, :]
        assert np.all(np.abs(got - want) <= 8 * 2.0 ** -24 * mag + 1e-30)
        return
    diff = got != want
    assert diff.mean() <= 2e-3, f"{int(diff.sum())} of {diff.size} differ"
    mbits = 10 if dtype == "f16" else 7
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(want), 1e-30))) - mbits)
    assert np.all(np.abs(got - want)[diff] <= ulp[diff])


def test_transform_hadamard_fast_rejects_other_dtypes():
    with pytest.raises(RuntimeError, match="dtype"):
        transform_hadamard_fast(torch.zeros((1, 128), dtype=torch.float64, device="cuda"))
    L = _lib.lib()
    assert L.exl3_hadamard_fast(None, None, None, 1, 128, 3, None) == _lib.EXL3_ERR_ARG
    assert L.exl3_hadamard_fast(None, None, None, 1, 100, 0, None) == _lib.EXL3_ERR_ARG


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
