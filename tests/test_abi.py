"""C ABI checks that need no GPU: the library loads, exports every entry point
include/sglang_exl3_amd.h declares, and rejects bad arguments with a status and
a message before touching the device."""

import ctypes
import os
import re

import pytest

from sglang_exl3 import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sglang_exl3_amd.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(exl3_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_entry_point():
    L = ctypes.CDLL(_lib.LIB_PATH)
    names = _declared()
    assert len(names) >= 8
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, f"not exported: {missing}"


def test_binding_table_covers_the_header():
    assert set(_declared()) == set(_lib.SIGNATURES), "ctypes signatures out of sync with the header"


def test_abi_version():
    assert _lib.lib().exl3_abi_version() == 1


@pytest.mark.parametrize("args,needle", [
    ((None, None, None, None, None, 0, 4096, 4096, 4, 1, None, 0, None), b"m=0"),
    ((None, None, None, None, None, 1, 4000, 4096, 4, 1, None, 0, None), b"multiples of 128"),
    ((None, None, None, None, None, 1, 4096, 4096, 9, 1, None, 0, None), b"K=9"),
    ((None, None, None, None, None, 1, 4096, 4096, 4, 3, None, 0, None), b"codebook=3"),
    ((None, None, None, None, None, 65, 4096, 4096, 4, 1, None, 0, None), b"m=65"),
    ((None, None, None, None, None, 1, 4096, 4096, 4, 1, None, 0, None), b"null pointer"),
])
def test_gemv_rejects_bad_arguments(args, needle):
    L = _lib.lib()
    assert L.exl3_gemv(*args) == _lib.EXL3_ERR_ARG
    assert needle in L.exl3_last_error()


def test_dequant_rejects_bad_arguments():
    L = _lib.lib()
    assert L.exl3_dequant_trellis(None, None, None, None, 128, 128, 4, 1, None) == _lib.EXL3_ERR_ARG
    assert L.exl3_dequant_trellis(1, 1, 1, 1, 100, 128, 4, 1, None) == _lib.EXL3_ERR_ARG
    assert b"k=100" in L.exl3_last_error()


def test_hadamard_fast_rejects_bad_arguments():
    L = _lib.lib()
    assert L.exl3_hadamard_fast(None, None, None, 1, 128, 3, None) == _lib.EXL3_ERR_ARG
    assert b"dtype=3" in L.exl3_last_error()
    assert L.exl3_hadamard_fast(None, None, None, 1, 100, _lib.DTYPE_BF16, None) == _lib.EXL3_ERR_ARG
    assert b"cols=100" in L.exl3_last_error()
    assert L.exl3_hadamard_fast(None, None, None, 2, 128, _lib.DTYPE_F32, None) == _lib.EXL3_ERR_ARG
    assert b"null pointer" in L.exl3_last_error()
    assert L.exl3_hadamard_fast(None, None, None, 0, 128, _lib.DTYPE_F16, None) == _lib.EXL3_OK


def test_batched_rejects_bad_arguments():
    L = _lib.lib()
    rc = L.exl3_p2b_gemv_batched(None, 0, None, None, None, None, 0, None, 1, 2048, 768, 3, 1, None, 0, None)
    assert rc == _lib.EXL3_ERR_ARG
    assert b"num_active" in L.exl3_last_error()


SK_STEPS = (1, 2, 3, 4, 5, 6, 7, 8, 10, 12, 14, 16)
SK_MAX_ROWS = 3  # rows served by the balanced kernel (kSkMaxRows in csrc/exl3_gemv.hip)


def _check_plan(m, k, n, K, experts=1):
    out = (ctypes.c_int * 5)()
    assert _lib.lib().exl3_gemv_plan(m, k, n, K, experts, out) == 0
    mb, ns, kw, splits, lds = list(out)
    assert 16 * mb >= m and 0 < lds <= 160 * 1024
    balanced = (experts == 1 and m <= SK_MAX_ROWS and m * n * 8 <= 4 * 1024 * 1024
                and os.environ.get("EXL3_GEMV_SK") != "0")
    if balanced:
        # balanced kernel: each column block's k/64 k-steps in `splits` equal pieces of ns steps
        ks_blk = k // 64
        assert kw == 1 and 1 <= splits <= min(63, ks_blk) and ks_blk % splits == 0
        assert ns == ks_blk // splits and ns in SK_STEPS
    else:
        # k-split kernel: k-slices covered exactly once, whole 128-row rotation blocks per workgroup
        assert 4 * ns * kw * splits == k // 16
        assert (4 * ns * kw) % 8 == 0
    return out


def test_workspace_and_plan_are_host_only():
    L = _lib.lib()
    # the balanced kernel needs the counter region plus one 8-byte accumulator per output
    assert L.exl3_gemv_workspace_size(1, 4096, 14336, 4, 1) >= 256 * 1024 + 14336 * 8
    _check_plan(1, 4096, 14336, 4)


@pytest.mark.parametrize("m,k,n,K", [(1, 128, 128, 1), (8, 768, 2048, 3), (16, 2048, 768, 3), (64, 256, 256, 2),
                                     (4, 4096, 1536, 5), (2, 14336, 4096, 4), (17, 1024, 512, 4)])
def test_plan_covers_k(m, k, n, K):
    _check_plan(m, k, n, K)
    _check_plan(m, k, n, K, experts=3)  # batched form: k-split kernel


def test_split_plan_when_balanced_disabled(monkeypatch):
    monkeypatch.setenv("EXL3_GEMV_SK", "0")
    out = _check_plan(1, 4096, 14336, 4)
    assert 4 * out[1] * out[2] * out[3] == 4096 // 16


def test_codebook_flag_mapping_matches_reference():
    # single-flag ops: mcg ? 1 : 2 (csrc/bindings.cpp:48); two-flag: none -> 3INST (0)
    assert _lib.codebook_from_mcg(True) == 1 and _lib.codebook_from_mcg(False) == 2
    assert _lib.codebook_id(False, False) == 0 and _lib.codebook_id(False, True) == 2
    with pytest.raises(ValueError):
        _lib.codebook_id(True, True)


def test_moe_plan_and_workspace_are_host_only():
    L = _lib.lib()
    out = (ctypes.c_int * 9)()
    for T in (1, 16, 64):
        assert L.exl3_moe_plan(T, 8, 128, 2048, 768, out) == 0
        gu, dn, units = list(out)[:4], list(out)[4:8], out[8]
        assert units == min(128, 8 * T) + (8 * T + 15) // 16  # bound on 16-row work units
        for (bpi, ns, kw, S), k, n in ((gu, 2048, 768), (dn, 768, 2048)):
            assert (n // 128) % bpi == 0
            assert 4 * ns * kw * S == k // 16
        assert L.exl3_moe_workspace_size(T, 8, 128, 2048, 768) > 256 * 1024
    assert L.exl3_moe_workspace_size(0, 8, 128, 2048, 768) == 0


def test_moe_plan_down_item_length(monkeypatch):
    """Down items of 12 steps (48 k-slices) where they leave one split with the fused combine
    (config 4, k = 768), 8-step items where 12 would leave two (config 5, k = 1536, 4 tokens);
    without the fused combine (above 48 tokens) 12 steps also with two splits."""
    for name in ("EXL3_MOE_DN_NSTEPS", "EXL3_MOE_NSTEPS", "EXL3_MOE_FC_TOKENS", "EXL3_MOE_FUSED_ROUTED"):
        monkeypatch.delenv(name, raising=False)
    L = _lib.lib()
    out = (ctypes.c_int * 9)()

    def down(T, topk, E, hidden, inter):
        assert L.exl3_moe_plan(T, topk, E, hidden, inter, out) == 0
        return out[5], out[7]  # steps, splits

    assert down(16, 8, 128, 2048, 768) == (12, 1)     # config 4, fused combine, one split
    assert down(4, 9, 289, 4096, 1536) == (8, 3)      # config 5: 8-step items, three splits
    assert down(64, 9, 289, 4096, 1536) == (12, 2)    # separate combine: two splits of 12 steps
    monkeypatch.setenv("EXL3_MOE_DN_NSTEPS", "12")    # the override still forces 12 steps
    assert down(4, 9, 289, 4096, 1536) == (12, 2)


def test_moe_rejects_bad_arguments_without_a_gpu():
    L = _lib.lib()
    nul = [None] * 9
    rc = L.exl3_moe_layer(None, None, None, *nul, 128, None, 1, 8, 2048, 768, 3, 3, 3, 1, 0.0, None, 0, None)
    assert rc == _lib.EXL3_ERR_ARG and b"null pointer" in L.exl3_last_error()
    rc = L.exl3_moe_layer(1, 1, 1, *([1] * 9), 128, 1, 1, 8, 2000, 768, 3, 3, 3, 1, 0.0, None, 0, None)
    assert rc == _lib.EXL3_ERR_ARG and b"multiples of 128" in L.exl3_last_error()
    rc = L.exl3_moe_layer(1, 1, 1, *([1] * 9), 5000, 1, 1, 8, 2048, 768, 3, 3, 3, 1, 0.0, None, 0, None)
    assert rc == _lib.EXL3_ERR_ARG and b"num_experts" in L.exl3_last_error()
    rc = L.exl3_moe_layer(4, 4, 4, *([4] * 9), 128, 4, 1, 8, 2048, 768, 3, 3, 3, 1, 0.0, None, 0, None)
    assert rc == _lib.EXL3_ERR_WORKSPACE
    rc = L.exl3_p2b_fused_moe(1, 1, *([1] * 9), 8, 1, 1, 4, 2048, 768, 3, 3, 9, 1, 0.0, None, 0, None)
    assert rc == _lib.EXL3_ERR_ARG and b"outside 1..8" in L.exl3_last_error()


@pytest.mark.parametrize("args,needle", [
    ((None, None, None, None, None, 0, 4096, 4096, 4, 1, None), b"m=0"),
    ((None, None, None, None, None, 65, 4096, 4096, 4, 1, None), b"m=65"),
    ((None, None, None, None, None, 1, 4000, 4096, 4, 1, None), b"multiples of 128"),
    ((None, None, None, None, None, 1, 4096, 4096, 0, 1, None), b"K=0"),
    ((None, None, None, None, None, 1, 4096, 4096, 4, 7, None), b"codebook=7"),
    ((None, None, None, None, None, 1, 4096, 4096, 4, 1, None), b"null pointer"),
])
def test_gemv_noalloc_rejects_bad_arguments_before_the_device(args, needle):
    L = _lib.lib()
    assert L.exl3_gemv_noalloc(*args) == _lib.EXL3_ERR_ARG
    assert needle in L.exl3_last_error()


def test_gemv_noalloc_refuses_shapes_beyond_its_scratch():
    L = _lib.lib()
    # 64 rows x 65536 columns need far more than the fixed 32 MiB (non-null dummy pointers: refused before use)
    assert L.exl3_gemv_workspace_size(64, 4096, 65536, 4, 1) > (32 << 20)
    rc = L.exl3_gemv_noalloc(16, 16, 16, 16, 16, 64, 4096, 65536, 4, 1, None)
    assert rc == _lib.EXL3_ERR_UNSUPPORTED
    assert b"above the fixed" in L.exl3_last_error()


def test_workspace_status_rejects_bad_arguments_without_a_gpu():
    import ctypes

    L = _lib.lib()
    st = ctypes.c_int32(0)
    assert L.exl3_workspace_status(None, 1 << 20, ctypes.byref(st), None) == _lib.EXL3_ERR_ARG
    assert b"null pointer" in L.exl3_last_error()
    assert L.exl3_workspace_status(16, 1 << 20, None, None) == _lib.EXL3_ERR_ARG
    assert L.exl3_workspace_status(16, 1024, ctypes.byref(st), None) == _lib.EXL3_ERR_ARG
    assert b"no status word" in L.exl3_last_error()
