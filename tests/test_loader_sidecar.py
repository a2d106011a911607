"""Checkpoint path on the CPU: safetensors streaming (reference
tests/test_mmap_loader.py) and routing of EXL3 groups onto per-shard linear
parameters (reference tests/test_sidecar_routing.py), then a synthetic
checkpoint streamed through both into EXL3LinearMethod layers."""

import json
import os
import struct

import numpy as np
import pytest
import torch
import torch.nn as nn
from safetensors.torch import load_file, save_file

from sglang_exl3.dense import EXL3LinearMethod
from sglang_exl3.exl3 import EXL3Config
from sglang_exl3.loader import (LOAD_FORMAT_EXL3_MMAP, EXL3MMapModelLoader, LoadFormatEXL3,
                                exl3_mmap_weights_iterator, is_unified_memory_platform, iter_safetensors_pread,
                                list_safetensors_shards, madvise_file_preload)
from sglang_exl3.sidecar import route_exl3_sidecar, split_fused_group, split_sidecar_name

# ----------------------------------------------------------------- loader


def test_loader_constants_and_platform():
    assert LoadFormatEXL3.EXL3_MMAP == LOAD_FORMAT_EXL3_MMAP == "exl3_mmap"
    assert is_unified_memory_platform() is False
    assert EXL3MMapModelLoader(load_config=None).load_format == "exl3_mmap"


def test_weights_iterator_two_shards(tmp_path):
    p1, p2 = str(tmp_path / "model-00001-of-00002.safetensors"), str(tmp_path / "model-00002-of-00002.safetensors")
    t1, t2, t3 = torch.randn(64, 128), torch.randn(128, 64), torch.randn(32, 32)
    save_file({"model.layers.0.weight": t1, "model.layers.0.bias": t2}, p1)
    save_file({"model.layers.1.weight": t3}, p2)
    assert madvise_file_preload(p1) in (True, False)
    got = dict(exl3_mmap_weights_iterator([p1, p2], device="cpu", num_threads=2, prefetch_shards=2))
    assert set(got) == {"model.layers.0.weight", "model.layers.0.bias", "model.layers.1.weight"}
    assert torch.equal(got["model.layers.0.weight"], t1)
    assert torch.equal(got["model.layers.0.bias"], t2)
    assert torch.equal(got["model.layers.1.weight"], t3)
    assert list(exl3_mmap_weights_iterator([])) == []


def test_pread_roundtrip_every_dtype(tmp_path):
    path = str(tmp_path / "m.safetensors")
    tensors = {
        "bf16": torch.randn(33, 17).to(torch.bfloat16),
        "f16": torch.randn(8, 16).to(torch.float16),
        "f32": torch.randn(5),
        "f64": torch.randn(3, dtype=torch.float64),
        "i8": torch.randint(-128, 127, (7,), dtype=torch.int8),
        "i16_trellis": torch.randint(-32768, 32767, (4, 16, 48), dtype=torch.int16),
        "i32": torch.arange(12, dtype=torch.int32).reshape(3, 4),
        "i64": torch.arange(5, dtype=torch.int64) - 2,
        "u8": torch.arange(256, dtype=torch.uint8),
        "bool": torch.tensor([True, False, True]),
        "scalar": torch.tensor(3, dtype=torch.int32),
        "empty": torch.empty(0, 4, dtype=torch.float16),
    }
    save_file(tensors, path, metadata={"format": "pt"})
    got = list(iter_safetensors_pread(path))
    names = [n for n, _ in got]
    assert set(names) == set(tensors)
    ref = load_file(path)
    for name, t in got:
        assert t.dtype == tensors[name].dtype and tuple(t.shape) == tuple(tensors[name].shape), name
        assert torch.equal(t, tensors[name]) and torch.equal(t, ref[name]), name
    # file order: ascending data offsets
    with open(path, "rb") as fh:
        (hlen,) = struct.unpack("<Q", fh.read(8))
        header = json.loads(fh.read(hlen))
    header.pop("__metadata__")
    assert names == sorted(header, key=lambda n: header[n]["data_offsets"][0])


def _write_raw(path, header, payload):
    h = json.dumps(header).encode()
    with open(path, "wb") as fh:
        fh.write(struct.pack("<Q", len(h)) + h + payload)


def test_pread_fails_closed(tmp_path):
    p = str(tmp_path / "bad.safetensors")
    _write_raw(p, {"x": {"dtype": "C64", "shape": [2], "data_offsets": [0, 16]}}, bytes(16))
    with pytest.raises(RuntimeError):
        list(iter_safetensors_pread(p))
    # byte range that does not match the shape
    _write_raw(p, {"x": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}, bytes(8))
    with pytest.raises(ValueError):
        list(iter_safetensors_pread(p))
    # data past the end of the file
    _write_raw(p, {"x": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}, bytes(8))
    with pytest.raises(ValueError):
        list(iter_safetensors_pread(p))
    # header length beyond the file
    with open(p, "wb") as fh:
        fh.write(struct.pack("<Q", 1 << 40) + b"{}")
    with pytest.raises(ValueError):
        list(iter_safetensors_pread(p))


def test_model_loader_without_sglang(tmp_path):
    save_file({"a": torch.ones(2)}, str(tmp_path / "model-00002-of-00002.safetensors"))
    save_file({"b": torch.zeros(3)}, str(tmp_path / "model-00001-of-00002.safetensors"))
    assert [os.path.basename(f) for f in list_safetensors_shards(str(tmp_path))] == [
        "model-00001-of-00002.safetensors", "model-00002-of-00002.safetensors"]

    class Src:
        model_or_path = str(tmp_path)
        revision = None
        fall_back_to_pt = False
        prefix = "m."

    loader = EXL3MMapModelLoader(load_config=None)
    got = dict(loader._get_weights_iterator(Src()))
    assert set(got) == {"m.a", "m.b"}
    with pytest.raises(FileNotFoundError):
        loader._prepare_weights(str(tmp_path / "nothing"), None, False)

# ---------------------------------------------------------------- sidecar


class _Owner:
    def __init__(self, sizes):
        self._exl3_lin_output_partition_sizes = list(sizes)


class _Param:
    def __init__(self, key, owner, sink):
        self.key, self._exl3_owner, self._sink = key, owner, sink

    def weight_loader(self, param, loaded, shard_id=None):
        self._sink.setdefault(self.key, []).append((shard_id, loaded.clone()))


_ALL = ("trellis", "suh", "svh", "mcg", "mul1")


def _params(base, n, sink, sizes):
    owner = _Owner(sizes)
    return {f"{base}.exl3_{i}_{s}": _Param(f"{base}.exl3_{i}_{s}", owner, sink) for i in range(n) for s in _ALL}


def test_split_sidecar_name():
    assert split_sidecar_name("a.b.trellis") == ("a.b", "trellis")
    assert split_sidecar_name("a.b.mul1") == ("a.b", "mul1")
    assert split_sidecar_name("a.b.weight") is None
    assert split_sidecar_name("trellis") is None


def test_fused_qkv_cut_along_output_tiles():
    sizes = [64, 32, 32]
    base = "model.layers.0.self_attn.qkv_proj"
    sink = {}
    params = _params(base, 3, sink, sizes)
    trellis = torch.arange(4 * 8 * 48, dtype=torch.int32).reshape(4, 8, 48).to(torch.int16)
    suh = torch.ones(64, dtype=torch.float16)
    svh = torch.arange(128, dtype=torch.float16)
    mul1 = torch.tensor(1, dtype=torch.int32)
    for name, t in ((base + ".trellis", trellis), (base + ".suh", suh), (base + ".svh", svh), (base + ".mul1", mul1)):
        assert route_exl3_sidecar(params, name, t), name
    assert torch.equal(sink[f"{base}.exl3_0_trellis"][0][1], trellis[:, 0:4, :])
    assert torch.equal(sink[f"{base}.exl3_1_trellis"][0][1], trellis[:, 4:6, :])
    assert torch.equal(sink[f"{base}.exl3_2_trellis"][0][1], trellis[:, 6:8, :])
    assert torch.equal(sink[f"{base}.exl3_1_svh"][0][1], svh[64:96])
    assert torch.equal(sink[f"{base}.exl3_2_svh"][0][1], svh[96:128])
    for i in range(3):
        assert torch.equal(sink[f"{base}.exl3_{i}_suh"][0][1], suh)
        assert sink[f"{base}.exl3_{i}_trellis"][0][0] == i
        assert sink[f"{base}.exl3_{i}_mul1"][0][1].item() == 1


def test_merged_gate_up_and_fused_qkv_a():
    sink = {}
    gu = "model.layers.5.mlp.shared_experts.gate_up_proj"
    params = _params(gu, 2, sink, [48, 48])
    t = torch.zeros(4, 3, 48, dtype=torch.int16)
    assert route_exl3_sidecar(params, "model.layers.5.mlp.shared_experts.gate_proj.trellis", t)
    assert route_exl3_sidecar(params, "model.layers.5.mlp.shared_experts.up_proj.trellis", t)
    assert sink[f"{gu}.exl3_0_trellis"][0][0] == 0 and sink[f"{gu}.exl3_1_trellis"][0][0] == 1
    fq = "model.layers.3.self_attn.fused_qkv_a_proj_with_mqa"
    sink2 = {}
    params2 = _params(fq, 2, sink2, [512, 64])
    assert route_exl3_sidecar(params2, "model.layers.3.self_attn.q_a_proj.svh", torch.zeros(512, dtype=torch.float16))
    assert route_exl3_sidecar(params2, "model.layers.3.self_attn.kv_a_proj_with_mqa.svh",
                              torch.zeros(64, dtype=torch.float16))
    assert sink2[f"{fq}.exl3_0_svh"][0][0] == 0 and sink2[f"{fq}.exl3_1_svh"][0][0] == 1
    # a merged leaf whose layer has one shard only: shard 1 does not exist
    params3 = _params("x.gate_up_proj", 1, {}, [32])
    with pytest.raises(RuntimeError):
        route_exl3_sidecar(params3, "x.up_proj.trellis", torch.zeros(1))


def test_single_shard_and_names_left_alone():
    sink = {}
    o = "model.layers.0.self_attn.o_proj"
    params = _params(o, 1, sink, [64])
    assert route_exl3_sidecar(params, o + ".trellis", torch.zeros(4, 4, 48, dtype=torch.int16))
    assert sink[f"{o}.exl3_0_trellis"][0][0] == 0
    assert not route_exl3_sidecar(params, "model.layers.0.mlp.experts.3.gate_proj.trellis", torch.zeros(1))
    assert not route_exl3_sidecar(params, o + ".weight", torch.zeros(1))
    assert not route_exl3_sidecar(params, "model.layers.9.self_attn.nope.trellis", torch.zeros(1))
    params[o + ".suh"] = object()  # a name the model owns directly is not a sidecar
    assert not route_exl3_sidecar(params, o + ".suh", torch.zeros(1))


def test_split_rejects_bad_sizes():
    with pytest.raises(ValueError):
        split_fused_group([24, 16], "svh", torch.zeros(40))
    with pytest.raises(ValueError):
        split_fused_group([32, 32], "trellis", torch.zeros(2, 3, 16))
    with pytest.raises(ValueError):
        split_fused_group([32, 32], "svh", torch.zeros(48))
    m = torch.tensor([1])
    assert all(p is m for p in split_fused_group([16, 32], "mcg", m))

# ------------------------------------------------- checkpoint -> layer packs


def _rand_group(rng, k, n, K):
    trellis = torch.from_numpy(rng.integers(-32768, 32767, size=(k // 16, n // 16, 16 * K), dtype=np.int16))
    suh = torch.from_numpy(np.where(rng.random(k) < 0.5, -1.0, 1.0).astype(np.float16))
    svh = torch.from_numpy((rng.standard_normal(n) * 0.01).astype(np.float16))
    return trellis, suh, svh


def build_checkpoint(tmp_path, K=3):
    """Two shards holding a fused qkv group, separate gate/up groups (merged
    layer) and a plain o_proj, with mcg markers; returns (files, groups)."""
    rng = np.random.default_rng(5)
    hidden, qkv, inter = 256, (256, 128, 128), 384  # 128-wide output blocks, as EXL3 packs them
    groups = {
        "model.layers.0.self_attn.qkv_proj": _rand_group(rng, hidden, sum(qkv), K),
        "model.layers.0.self_attn.o_proj": _rand_group(rng, 128, hidden, K),
        "model.layers.0.mlp.gate_proj": _rand_group(rng, hidden, inter, K),
        "model.layers.0.mlp.up_proj": _rand_group(rng, hidden, inter, K),
    }
    shard1, shard2 = {}, {}
    for j, (mod, (t, su, sv)) in enumerate(groups.items()):
        dst = shard1 if j < 2 else shard2
        dst[mod + ".trellis"], dst[mod + ".suh"], dst[mod + ".svh"] = t, su, sv
        dst[mod + ".mcg"] = torch.tensor(1, dtype=torch.int32)
    shard2["model.norm.weight"] = torch.ones(hidden, dtype=torch.bfloat16)  # not EXL3
    files = [str(tmp_path / "model-00001-of-00002.safetensors"), str(tmp_path / "model-00002-of-00002.safetensors")]
    save_file(shard1, files[0])
    save_file(shard2, files[1])
    return files, groups, (hidden, qkv, inter)


def load_layers(files, dims):
    """Stream the checkpoint into EXL3LinearMethod layers through the sidecar router."""
    hidden, qkv, inter = dims
    cfg = EXL3Config.from_config({"bits": 3, "codebook": "mcg"})
    specs = {
        "model.layers.0.self_attn.qkv_proj": (hidden, list(qkv)),
        "model.layers.0.self_attn.o_proj": (128, [hidden]),
        "model.layers.0.mlp.gate_up_proj": (hidden, [inter, inter]),
    }
    layers, params = {}, {}
    for prefix, (k, outs) in specs.items():
        layer = nn.Module()
        EXL3LinearMethod(cfg, bits=3).create_weights(layer, k, outs, k, sum(outs), torch.float16)
        layers[prefix] = layer
        for name, p in layer.named_parameters():
            params[f"{prefix}.{name}"] = p
    leftovers = []
    for name, tensor in exl3_mmap_weights_iterator(files):
        if not route_exl3_sidecar(params, name, tensor):
            leftovers.append(name)
    return layers, leftovers


def test_checkpoint_streams_into_layer_packs(tmp_path):
    files, groups, dims = build_checkpoint(tmp_path)
    layers, leftovers = load_layers(files, dims)
    assert leftovers == ["model.norm.weight"]
    qkv = layers["model.layers.0.self_attn.qkv_proj"]._exl3_lin_packs
    t, su, sv = groups["model.layers.0.self_attn.qkv_proj"]
    cuts = [0, 16, 24, 32]
    for i in range(3):
        assert torch.equal(qkv[i]["trellis"].cpu(), t[:, cuts[i]:cuts[i + 1], :])
        assert torch.equal(qkv[i]["svh"].cpu(), sv[cuts[i] * 16:cuts[i + 1] * 16])
        assert torch.equal(qkv[i]["suh"].cpu(), su)
        assert int(qkv[i]["mcg"].item()) == 1
    gu = layers["model.layers.0.mlp.gate_up_proj"]._exl3_lin_packs
    for i, mod in enumerate(("model.layers.0.mlp.gate_proj", "model.layers.0.mlp.up_proj")):
        for j, key in enumerate(("trellis", "suh", "svh")):
            assert torch.equal(gu[i][key].cpu(), groups[mod][j])
    # every shard complete -> the linears build, K from the trellis shape
    for layer in layers.values():
        EXL3LinearMethod(EXL3Config.from_config({"bits": 3}), bits=3).process_weights_after_loading(layer)
        assert all(lin.K == 3 and lin.mcg for lin in layer._exl3_linears)
