"""sglang_exl3 — MI355X (gfx950) EXL3 quantized-matmul path for SGLang.

Keeps the reference plugin's public surface (src/sglang_exl3/__init__.py:33-63):
``register()`` registers the ``torch.ops.sglang_exl3.*`` custom ops (and the
SGLang quantization method when SGLang is importable).  The ops are backed by
the C-ABI HIP library ``_lib/libsglang_exl3_amd.so``.
"""

from __future__ import annotations

import logging

logger = logging.getLogger("sglang.exl3")

__all__ = ["register"]


def register() -> None:
    """Register the custom ops and, when SGLang is present, the "exl3" quantization method."""
    from . import ops

    ops.register_custom_ops()
    try:  # SGLang is optional: the plugin surface works without it
        from sglang.srt.layers.quantization import QUANTIZATION_METHODS  # type: ignore

        from .exl3 import EXL3Config

        QUANTIZATION_METHODS.setdefault("exl3", EXL3Config)
    except Exception:  # noqa: BLE001 - SGLang absent or incompatible
        pass
