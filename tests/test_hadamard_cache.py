"""HadamardPrefixCache behaviour (CPU), mirroring the reference's
tests/test_hadamard_cache.py:34-94, and the oracle's row transform pinned
against the Sylvester matrix."""

import os

import numpy as np
import pytest
import torch

import oracle
from sglang_exl3.hadamard_cache import (
    OPT_MOE_QUANT_ONCE_ENV,
    HadamardPrefixCache,
    get_global_hadamard_cache,
    is_moe_quant_once_enabled,
)


def test_cache_store_lookup_and_slicing():
    cache = HadamardPrefixCache(max_entries=4)
    h, layer = 0xABCD1234, 5
    data = torch.randn((128, 4096), dtype=torch.float16)
    cache.put(h, layer, data)
    hit = cache.get(h, layer, 128)
    assert hit is not None and hit.shape == (128, 4096)
    torch.testing.assert_close(hit, data)
    part = cache.get(h, layer, 64)
    assert part is not None and part.shape == (64, 4096)
    torch.testing.assert_close(part, data[:64])
    assert cache.get(h, layer, 256) is None  # longer than stored
    assert cache.get(h, 6, 128) is None      # other layer
    assert cache.get(0x99999999, layer, 128) is None
    assert cache.hits == 2 and cache.misses == 3 and cache.hit_rate == pytest.approx(0.4)


def test_lru_eviction():
    cache = HadamardPrefixCache(max_entries=2)
    cache.put(1, 0, torch.zeros((10, 128)))
    cache.put(2, 0, torch.zeros((10, 128)))
    assert cache.get(1, 0, 10) is not None  # 1 becomes most recent
    cache.put(3, 0, torch.zeros((10, 128)))  # evicts 2
    assert cache.get(1, 0, 10) is not None
    assert cache.get(2, 0, 10) is None
    assert cache.get(3, 0, 10) is not None
    assert len(cache) == 2
    cache.clear()
    assert len(cache) == 0 and cache.hits == 0 and cache.hit_rate == 0.0


def test_env_toggle(monkeypatch):
    monkeypatch.setenv(OPT_MOE_QUANT_ONCE_ENV, "0")
    assert not is_moe_quant_once_enabled()
    cache = HadamardPrefixCache()
    cache.put(1, 0, torch.zeros((10, 128)))
    assert cache.get(1, 0, 10) is None
    monkeypatch.setenv(OPT_MOE_QUANT_ONCE_ENV, "yes")
    assert is_moe_quant_once_enabled()
    assert get_global_hadamard_cache() is get_global_hadamard_cache()


def test_oracle_had_rows_is_the_matrix_product():
    """oracle.had_rows = ((x * pre) @ H) * r * post per 128 block (H symmetric)."""
    H = np.array([[1.0]])
    while H.shape[0] < 128:
        H = np.block([[H, H], [H, -H]])
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 256)).astype(np.float32)
    pre = rng.choice([-1.0, 0.5, 2.0], 256).astype(np.float16)
    post = rng.choice([-1.0, 0.25, 1.0], 256).astype(np.float16)
    r = 0.0883883476
    y = oracle.had_rows(x, pre, post, r)
    want = np.zeros_like(y, dtype=np.float64)
    for c0 in (0, 128):
        blk = x[:, c0:c0 + 128].astype(np.float64) * pre[c0:c0 + 128].astype(np.float64)
        want[:, c0:c0 + 128] = (blk @ H) * r * post[c0:c0 + 128].astype(np.float64)
    assert np.allclose(y, want, rtol=1e-5, atol=1e-4)
    assert np.allclose(oracle.had_rows(oracle.had_rows(x, None, None, r), None, None, r), x, atol=1e-5)
