"""Prefix-keyed cache of Hadamard-rotated activations and the row Hadamard
transform that fills it.

Same surface as the reference module (src/sglang_exl3/hadamard_cache.py:1-120):
``HadamardPrefixCache`` (LRU keyed by (prefix_hash, layer_id), prefix slicing,
hit/miss counters, gated by SGLANG_OPT_MOE_QUANT_ONCE), the process-wide
instance, and ``transform_hadamard_fast`` (rows in blocks of 128, normalised
Hadamard, optional post-scale by suh).  The transform runs the gfx950 kernel
behind ``exl3_hadamard_fast`` in x's dtype (fp16, bf16, fp32) with the
reference's scale and roundings; only the order of the fp32 block sum differs
from the reference's matmul.  ``hadamard_rows`` is the fp16 row transform with
pre/post scales that the expert paths use (exllamav3's had_r_128).
"""

from __future__ import annotations

import collections
import logging
import os
from typing import Optional, Tuple

import torch

from . import _lib

logger = logging.getLogger("sglang.exl3.hadamard_cache")

OPT_MOE_QUANT_ONCE_ENV = "SGLANG_OPT_MOE_QUANT_ONCE"
MAX_CACHE_ENTRIES_DEFAULT = 128
HAD_NORM = 0.08838834764831845  # 1/sqrt(128)


def is_moe_quant_once_enabled() -> bool:
    """Caching is on unless SGLANG_OPT_MOE_QUANT_ONCE is set to something other than 1/true/yes/on."""
    return os.environ.get(OPT_MOE_QUANT_ONCE_ENV, "1").strip().lower() in {"1", "true", "yes", "on"}


class HadamardPrefixCache:
    """LRU of rotated activations keyed by (prefix_hash, layer_id).

    ``get(h, layer, n)`` returns the first n rows of the stored tensor when it has
    at least n rows (a shared prefix), else None; ``put`` stores (detached) and
    evicts the least recently used entry beyond ``max_entries``."""

    def __init__(self, max_entries: int = MAX_CACHE_ENTRIES_DEFAULT):
        self.max_entries = int(max_entries)
        self._entries: "collections.OrderedDict[Tuple[int, int], torch.Tensor]" = collections.OrderedDict()
        self.hits = 0
        self.misses = 0

    def get(self, prefix_hash: Optional[int], layer_id: int, prefix_len: int) -> Optional[torch.Tensor]:
        if not is_moe_quant_once_enabled() or prefix_hash is None or prefix_len <= 0:
            return None
        key = (prefix_hash, layer_id)
        t = self._entries.get(key)
        if t is not None and t.shape[0] >= prefix_len:
            self._entries.move_to_end(key)
            self.hits += 1
            return t[:prefix_len]
        self.misses += 1
        return None

    def put(self, prefix_hash: Optional[int], layer_id: int, transformed: torch.Tensor) -> None:
        if not is_moe_quant_once_enabled() or prefix_hash is None:
            return
        key = (prefix_hash, layer_id)
        if key in self._entries:
            self._entries.move_to_end(key)
        else:
            while self._entries and len(self._entries) >= self.max_entries:
                self._entries.popitem(last=False)
        self._entries[key] = transformed.detach()

    def clear(self) -> None:
        self._entries.clear()
        self.hits = 0
        self.misses = 0

    @property
    def hit_rate(self) -> float:
        n = self.hits + self.misses
        return self.hits / n if n else 0.0

    def __len__(self) -> int:
        return len(self._entries)


_GLOBAL_CACHE = HadamardPrefixCache()


def get_global_hadamard_cache() -> HadamardPrefixCache:
    return _GLOBAL_CACHE


def hadamard_rows(x: torch.Tensor, pre: Optional[torch.Tensor] = None, post: Optional[torch.Tensor] = None,
                  scale: float = HAD_NORM, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = fp16(H(x * pre) * scale * post) per 128-column block of the last dim
    (H unnormalised; the default scale normalises).  fp16 HIP tensors only."""
    if not x.is_cuda:
        raise RuntimeError("sglang_exl3 hadamard_rows requires HIP device tensors")
    if x.dtype != torch.float16:
        raise RuntimeError("sglang_exl3 hadamard_rows: x must be float16")
    cols = int(x.shape[-1])
    if cols % 128:
        raise RuntimeError("sglang_exl3 hadamard_rows: last dim must be a multiple of 128")
    xc = x.contiguous()
    rows = xc.numel() // cols if cols else 0
    y = torch.empty_like(xc) if out is None else out
    if y.dtype != torch.float16 or not y.is_contiguous() or y.shape != xc.shape:
        raise RuntimeError("sglang_exl3 hadamard_rows: out must be a contiguous fp16 tensor shaped like x")
    vecs = []
    for v in (pre, post):
        if v is None:
            vecs.append(None)
            continue
        if v.dtype != torch.float16 or v.numel() != cols or v.device != x.device:
            raise RuntimeError("sglang_exl3 hadamard_rows: pre/post must be fp16 vectors of the last dim")
        vecs.append(v.contiguous())
    with torch.cuda.device(x.device):
        rc = _lib.lib().exl3_hadamard_rows(
            xc.data_ptr(), y.data_ptr(), None if vecs[0] is None else vecs[0].data_ptr(),
            None if vecs[1] is None else vecs[1].data_ptr(), float(scale), rows, cols,
            int(torch.cuda.current_stream(x.device).cuda_stream))
    _lib.check(rc, "exl3_hadamard_rows")
    return y


_FAST_DTYPES = {torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16, torch.float32: _lib.DTYPE_F32}


def transform_hadamard_fast(x: torch.Tensor, suh: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Row-wise normalised Walsh-Hadamard transform in blocks of 128, then the
    optional suh product, in x's dtype (src/sglang_exl3/hadamard_cache.py:88-120):
    the block sums are scaled by 1/sqrt(128) rounded to that dtype and rounded
    to it, then multiplied by suh converted to it and rounded again, as the
    reference's matmul by its cached matrix and its suh product do.  Widths
    that are not multiples of 128 come back unchanged, as in the reference.
    fp16, bf16 and fp32 HIP tensors."""
    hidden = int(x.shape[-1])
    if hidden % 128:
        return x
    code = _FAST_DTYPES.get(x.dtype)
    if code is None:
        raise RuntimeError(f"sglang_exl3 transform_hadamard_fast: dtype {x.dtype} (fp16, bf16 or fp32)")
    if not x.is_cuda:
        raise RuntimeError("sglang_exl3 transform_hadamard_fast requires HIP device tensors")
    post = None
    if suh is not None and suh.numel() == hidden:
        post = suh.reshape(-1).to(device=x.device, dtype=x.dtype).contiguous()
    xc = x.reshape(-1, hidden).contiguous()
    y = torch.empty_like(xc)
    with torch.cuda.device(x.device):
        rc = _lib.lib().exl3_hadamard_fast(xc.data_ptr(), y.data_ptr(), None if post is None else post.data_ptr(),
                                           int(xc.shape[0]), hidden, code,
                                           int(torch.cuda.current_stream(x.device).cuda_stream))
    _lib.check(rc, "exl3_hadamard_fast")
    return y.view_as(x)
