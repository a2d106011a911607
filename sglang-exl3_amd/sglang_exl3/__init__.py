"""sglang_exl3 — MI355X (gfx950) EXL3 quantized-matmul path for SGLang.

Keeps the reference plugin's public surface (src/sglang_exl3/__init__.py:33-63):
``register()`` registers the ``torch.ops.sglang_exl3.*`` custom ops and, when
SGLang is importable, the "exl3" quantization method, its CLI choice and the
"exl3_mmap" load format (patch.py).  The ops are backed by the C-ABI HIP
library ``_lib/libsglang_exl3_amd.so``.
"""

from __future__ import annotations

import logging

logger = logging.getLogger("sglang.exl3")

__all__ = ["register"]


def register() -> bool:
    """Register the custom ops and the SGLang integration; returns whether any
    SGLang table was patched (False when SGLang is not installed)."""
    from . import ops, patch

    ops.register_custom_ops()
    return patch.apply_all_patches()
