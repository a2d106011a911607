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


def test_batched_rejects_bad_arguments():
    L = _lib.lib()
    rc = L.exl3_p2b_gemv_batched(None, 0, None, None, None, None, 0, None, 1, 2048, 768, 3, 1, None, 0, None)
    assert rc == _lib.EXL3_ERR_ARG
    assert b"num_active" in L.exl3_last_error()


def test_workspace_and_plan_are_host_only():
    L = _lib.lib()
    assert L.exl3_gemv_workspace_size(1, 4096, 14336, 4, 1) > 0
    out = (ctypes.c_int * 5)()
    assert L.exl3_gemv_plan(1, 4096, 14336, 4, 1, out) == 0
    mb, ns, kw, splits, lds = list(out)
    assert mb == 1 and ns in (2, 4, 8, 16) and kw in (1, 2)
    assert 4 * ns * kw * splits == 4096 // 16  # k-slices covered exactly once
    assert 0 < lds <= 160 * 1024


@pytest.mark.parametrize("m,k,n,K", [(1, 128, 128, 1), (8, 768, 2048, 3), (16, 2048, 768, 3), (64, 256, 256, 2),
                                     (4, 4096, 1536, 5), (2, 14336, 4096, 4)])
def test_plan_covers_k_exactly(m, k, n, K):
    out = (ctypes.c_int * 5)()
    assert _lib.lib().exl3_gemv_plan(m, k, n, K, 1, out) == 0
    mb, ns, kw, splits, lds = list(out)
    assert 16 * mb >= m
    assert 4 * ns * kw * splits == k // 16
    assert (4 * ns * kw) % 8 == 0  # whole 128-row rotation blocks per workgroup


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
