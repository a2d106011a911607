"""register() / patch.py against SGLang's tables (reference tests/test_registration.py).

SGLang is not installed here, so the tests put a minimal stand-in module tree
under ``sys.modules["sglang"]`` holding exactly the attributes the patches
touch, run register(), and check each table; without the stand-in register()
still registers the ops and reports that nothing was patched."""

import sys
import types

import pytest

import sglang_exl3
from sglang_exl3 import patch
from sglang_exl3.exl3 import EXL3Config
from sglang_exl3.loader import EXL3MMapModelLoader


def _fake_sglang(monkeypatch, with_adder=False):
    mods = {}
    for name in ("sglang", "sglang.srt", "sglang.srt.layers", "sglang.srt.layers.quantization",
                 "sglang.srt.configs", "sglang.srt.configs.model_config", "sglang.srt.configs.load_config",
                 "sglang.srt.server_args", "sglang.srt.model_loader", "sglang.srt.model_loader.loader"):
        mods[name] = types.ModuleType(name)
    q = mods["sglang.srt.layers.quantization"]
    q.QUANTIZATION_METHODS = {"fp8": object}
    q.BASE_QUANTIZATION_METHODS = {"fp8": object}
    mods["sglang.srt.configs.model_config"].QUANTIZATION_METHODS = {"fp8": object}
    sa = mods["sglang.srt.server_args"]
    sa.QUANTIZATION_CHOICES = ["fp8"]
    sa.LOAD_FORMAT_CHOICES = ["auto", "safetensors"]
    if with_adder:
        sa.added = []
        sa.add_quantization_method_choices = lambda names: (sa.added.extend(names), sa.QUANTIZATION_CHOICES.extend(names))

    class LoadConfig:
        def __init__(self, load_format):
            self.load_format = load_format
            self._verify_load_format()

        def _verify_load_format(self):
            if self.load_format not in ("auto", "safetensors"):
                raise ValueError(f"unknown load format {self.load_format}")

    mods["sglang.srt.configs.load_config"].LoadConfig = LoadConfig
    sentinel = object()
    mods["sglang.srt.model_loader.loader"].get_model_loader = lambda load_config, model_config=None: sentinel
    # parent packages expose their children as attributes, as real packages do
    for name, mod in mods.items():
        parent, _, leaf = name.rpartition(".")
        if parent:
            setattr(mods[parent], leaf, mod)
        monkeypatch.setitem(sys.modules, name, mod)
    return mods, sentinel


def test_register_patches_sglang_tables(monkeypatch):
    mods, sentinel = _fake_sglang(monkeypatch)
    assert sglang_exl3.register() is True
    assert mods["sglang.srt.layers.quantization"].QUANTIZATION_METHODS["exl3"] is EXL3Config
    assert mods["sglang.srt.layers.quantization"].BASE_QUANTIZATION_METHODS["exl3"] is EXL3Config
    assert mods["sglang.srt.configs.model_config"].QUANTIZATION_METHODS["exl3"] is EXL3Config
    sa = mods["sglang.srt.server_args"]
    assert sa.QUANTIZATION_CHOICES.count("exl3") == 1 and "exl3_mmap" in sa.LOAD_FORMAT_CHOICES
    LoadConfig = mods["sglang.srt.configs.load_config"].LoadConfig
    lc = LoadConfig("EXL3_MMAP")  # accepted (case-insensitive) and normalised
    assert lc.load_format == "exl3_mmap"
    with pytest.raises(ValueError):
        LoadConfig("bogus")  # other formats keep the original check
    sml = mods["sglang.srt.model_loader.loader"]
    assert isinstance(sml.get_model_loader(lc), EXL3MMapModelLoader)
    assert sml.get_model_loader(LoadConfig("auto")) is sentinel
    # idempotent: a second register() adds nothing twice and does not re-wrap
    loader_fn = sml.get_model_loader
    assert sglang_exl3.register() is True
    assert sa.QUANTIZATION_CHOICES.count("exl3") == 1 and sa.LOAD_FORMAT_CHOICES.count("exl3_mmap") == 1
    assert sml.get_model_loader is loader_fn


def test_server_args_uses_the_adder_when_present(monkeypatch):
    mods, _ = _fake_sglang(monkeypatch, with_adder=True)
    assert patch.patch_server_args()
    assert mods["sglang.srt.server_args"].added == ["exl3"]


def test_register_without_sglang(monkeypatch):
    for name in [n for n in sys.modules if n == "sglang" or n.startswith("sglang.")]:
        monkeypatch.delitem(sys.modules, name)
    monkeypatch.setitem(sys.modules, "sglang", None)  # import sglang -> ImportError
    assert sglang_exl3.register() is False
    assert not patch.patch_quantization_methods()
    assert not patch.patch_server_args()
    assert not patch.patch_model_loader()
