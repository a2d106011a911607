"""SGLang base classes when SGLang is installed, minimal stand-ins otherwise.

The quantization config and methods subclass these so that the same objects
plug into SGLang's loader when it is present and stay usable (and testable)
without it.
"""

from __future__ import annotations

from typing import Any

import torch
from torch.nn.parameter import Parameter

try:  # pragma: no cover - depends on SGLang being installed
    from sglang.srt.layers.quantization.base_config import (  # type: ignore
        FusedMoEMethodBase,
        LinearMethodBase,
        QuantizationConfig,
        QuantizeMethodBase,
    )

    HAVE_SGLANG = True
except Exception:  # noqa: BLE001
    HAVE_SGLANG = False

    class QuantizeMethodBase:  # type: ignore[no-redef]
        def create_weights(self, layer: torch.nn.Module, *args, **kwargs):
            raise NotImplementedError

        def apply(self, layer: torch.nn.Module, *args, **kwargs):
            raise NotImplementedError

        def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
            return None

    class LinearMethodBase(QuantizeMethodBase):  # type: ignore[no-redef]
        pass

    class FusedMoEMethodBase(QuantizeMethodBase):  # type: ignore[no-redef]
        runner = None

        def create_moe_runner(self, layer: torch.nn.Module, moe_runner_config: Any):
            self.runner = None

    class QuantizationConfig:  # type: ignore[no-redef]
        def __init__(self):
            self.packed_modules_mapping = {}

        def update_packed_modules_mapping(self, mapping):
            self.packed_modules_mapping = mapping


def set_weight_attrs(param: Parameter, extra_attrs: dict) -> None:
    """SGLang's set_weight_attrs when available, else plain setattr."""
    try:  # pragma: no cover - SGLang present
        from sglang.srt.utils import set_weight_attrs as _sgl  # type: ignore

        _sgl(param, extra_attrs)
        return
    except Exception:  # noqa: BLE001
        pass
    for k, v in (extra_attrs or {}).items():
        setattr(param, k, v)


def unquantized_linear_method():
    """SGLang's UnquantizedLinearMethod, or None (= leave the layer as it is)."""
    try:  # pragma: no cover - SGLang present
        from sglang.srt.layers.quantization.unquant import UnquantizedLinearMethod  # type: ignore

        return UnquantizedLinearMethod()
    except Exception:  # noqa: BLE001
        return None
