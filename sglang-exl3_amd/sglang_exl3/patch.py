"""Registration of the EXL3 plugin into SGLang's tables (reference:
src/sglang_exl3/patch.py:13-52 and 162-242).

Each patch is idempotent and returns False, without raising, when SGLang (or
the piece it patches) is not importable:

- ``patch_quantization_methods``: "exl3" -> EXL3Config in SGLang's quantization
  method tables (also the copy model_config imported);
- ``patch_server_args``: "exl3" among the ``--quantization`` choices;
- ``patch_model_loader``: the "exl3_mmap" load format (LoadConfig accepts it,
  ``get_model_loader`` returns EXL3MMapModelLoader for it, and it is a
  ``--load-format`` choice).

The reference's model-specific patches (DeepSeek-V4 weight filtering, DSpark
draft gamma) belong to model families outside the EXL3 matmul path and are
not carried.
"""

from __future__ import annotations

import logging

logger = logging.getLogger("sglang.exl3")


def patch_quantization_methods() -> bool:
    try:
        from sglang.srt.layers import quantization as sq  # type: ignore

        from .exl3 import EXL3Config
    except (ImportError, AttributeError) as exc:
        logger.debug("EXL3: SGLang quantization table not patched: %s", exc)
        return False
    for table in ("QUANTIZATION_METHODS", "BASE_QUANTIZATION_METHODS"):
        methods = getattr(sq, table, None)
        if isinstance(methods, dict):
            methods["exl3"] = EXL3Config
    try:
        from sglang.srt.configs import model_config as smc  # type: ignore

        methods = getattr(smc, "QUANTIZATION_METHODS", None)
        if isinstance(methods, dict):
            methods["exl3"] = EXL3Config
    except (ImportError, AttributeError):
        pass
    return True


def patch_server_args() -> bool:
    try:
        from sglang.srt import server_args as sa  # type: ignore
    except (ImportError, AttributeError) as exc:
        logger.debug("EXL3: SGLang server args not patched: %s", exc)
        return False
    choices = getattr(sa, "QUANTIZATION_CHOICES", None)
    if choices is not None and "exl3" not in choices:
        adder = getattr(sa, "add_quantization_method_choices", None)
        if callable(adder):
            adder(["exl3"])
        else:
            choices.append("exl3")
    return True


def patch_model_loader() -> bool:
    try:
        from sglang.srt.model_loader import loader as sml  # type: ignore

        from .loader import LOAD_FORMAT_EXL3_MMAP, EXL3MMapModelLoader
    except (ImportError, AttributeError) as exc:
        logger.debug("EXL3: SGLang model loader not patched: %s", exc)
        return False
    # LoadConfig validates string formats against its enum before a loader is
    # chosen: accept ours there, leave every other format to the original check
    try:
        from sglang.srt.configs.load_config import LoadConfig  # type: ignore

        if not getattr(LoadConfig, "_exl3_mmap_patched", False) and hasattr(LoadConfig, "_verify_load_format"):
            verify = LoadConfig._verify_load_format

            def _verify_load_format(self):
                if isinstance(self.load_format, str) and self.load_format.lower() == LOAD_FORMAT_EXL3_MMAP:
                    self.load_format = LOAD_FORMAT_EXL3_MMAP
                    return None
                return verify(self)

            LoadConfig._verify_load_format = _verify_load_format
            LoadConfig._exl3_mmap_patched = True
    except (ImportError, AttributeError):
        pass
    get_loader = getattr(sml, "get_model_loader", None)
    if callable(get_loader) and not getattr(get_loader, "_exl3_patched", False):
        def get_model_loader(load_config, *args, **kwargs):
            if getattr(load_config, "load_format", None) == LOAD_FORMAT_EXL3_MMAP:
                return EXL3MMapModelLoader(load_config)
            return get_loader(load_config, *args, **kwargs)

        get_model_loader._exl3_patched = True
        sml.get_model_loader = get_model_loader
    try:
        from sglang.srt import server_args as sa  # type: ignore

        formats = getattr(sa, "LOAD_FORMAT_CHOICES", None)
        if formats is not None and LOAD_FORMAT_EXL3_MMAP not in formats:
            formats.append(LOAD_FORMAT_EXL3_MMAP)
    except (ImportError, AttributeError):
        pass
    return True


def apply_all_patches() -> bool:
    """Every patch above; True when at least one applied."""
    results = [patch_quantization_methods(), patch_server_args(), patch_model_loader()]
    return any(results)
