"""torch.ops.sglang_exl3 registry and fake-tensor shape inference (CPU).

Mirrors the reference's tests/test_cuda_graph.py:13-68 (same op list, same fake
shapes), and checks that CPU tensors are refused (no CPU fallback)."""

import pytest
import torch

import sglang_exl3
from sglang_exl3 import ops


@pytest.fixture(scope="module", autouse=True)
def _registered():
    sglang_exl3.register()
    ops.register_custom_ops()


def test_ops_registered_in_torch():
    for name in ops.OP_NAMES:
        assert hasattr(torch.ops.sglang_exl3, name), name


def test_meta_fake_tensor_dispatch():
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        x = torch.empty((2, 128), dtype=torch.float16)
        trellis = torch.empty((8, 16, 32), dtype=torch.int16)
        suh = torch.empty((128,), dtype=torch.float16)
        svh = torch.empty((256,), dtype=torch.float16)
        g = torch.ops.sglang_exl3.exl3_gemv(x, trellis, suh, svh, 2, True, 1)
        assert g.shape == (2, 256) and g.dtype == torch.float16
        gm = torch.ops.sglang_exl3.exl3_gemm(x, trellis, suh, svh, 2, True)
        assert gm.shape == (2, 256) and gm.dtype == torch.float16
        d = torch.ops.sglang_exl3.dequant_trellis(trellis, suh, svh, 2, True)
        assert d.shape == (128, 256) and d.dtype == torch.float16
        ptrs = torch.empty((4,), dtype=torch.int64)
        ids = torch.empty((6,), dtype=torch.int32)
        b = torch.ops.sglang_exl3.p2b_gemv_batched(x, ptrs, ptrs, ptrs, ids, 2, True, 768)
        assert b.shape == (6, 2, 768)
        b2 = torch.ops.sglang_exl3.p2b_gemv_batched(x, ptrs, ptrs, ptrs, ids, 2, True, 0)
        assert b2.shape == (6, 2, 2048)
        out = torch.empty((1, 128), dtype=torch.float16)
        w = torch.empty((6,), dtype=torch.float16)
        assert torch.ops.sglang_exl3.p2b_fused_moe(x[:1], out, ptrs, ptrs, ptrs, ptrs, ptrs, ptrs, ptrs, ptrs,
                                                   ptrs, ids, w, 2, 2, 2, True) is None
        o32 = torch.empty((2, 256), dtype=torch.float32)
        assert torch.ops.sglang_exl3.exl3_fat_gemm(x, trellis, o32, svh, 2, True, False) is None


def test_cpu_tensors_are_refused():
    x = torch.zeros((1, 128), dtype=torch.float16)
    trellis = torch.zeros((8, 16, 32), dtype=torch.int16)
    suh = torch.ones(128, dtype=torch.float16)
    svh = torch.ones(256, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="HIP device"):
        torch.ops.sglang_exl3.exl3_gemv(x, trellis, suh, svh, 2, True, 1)
    with pytest.raises(RuntimeError, match="HIP device"):
        torch.ops.sglang_exl3.dequant_trellis(trellis, suh, svh, 2, True)
