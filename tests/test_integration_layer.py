"""Config, routing and method plumbing of the SGLang integration layer (CPU).

Mirrors the reference's tests/test_config.py, test_tensor_storage_kinds.py,
test_dense_marker_codebook.py, test_moe.py (weight creation, map_topk_to_local),
test_fused_moe_k.py (per-projection K) and test_python_loop_capture_guard.py.
"""

from unittest import mock

import pytest
import torch
import torch.nn as nn

from sglang_exl3 import exl3
from sglang_exl3.dense import EXL3DenseLinear, EXL3LinearMethod
from sglang_exl3.exl3 import (
    MCG_MARKER_SIGNED_INT32,
    MUL1_MARKER_SIGNED_INT32,
    EXL3Config,
    EXL3MoEMethod,
    _tensor_storage_bits,
    _tensor_storage_kinds,
    build_exl3_fused_state,
    map_topk_to_local,
    shard_exl3_col,
    shard_exl3_row,
)


# ------------------------------------------------------------------- config

def test_default_config():
    cfg = EXL3Config(bits=4, codebook="mcg")
    assert cfg.get_name() == "exl3" and cfg.bits == 4 and cfg.codebook == "mcg"
    assert cfg.get_min_capability() == 80
    with pytest.raises(ValueError):
        EXL3Config(bits=7)
    with pytest.raises(ValueError):
        EXL3Config(codebook="3inst")


def test_mixed_k_layer_bits():
    cfg = EXL3Config(bits=2, layer_bits={"42": 3, "27": 3})
    assert cfg.bits_for_prefix("model.layers.0.mlp.experts") == 2
    assert cfg.bits_for_prefix("model.layers.42.mlp.experts") == 3
    assert cfg.bits_for_prefix("model.layers.27.mlp.experts") == 3


def test_from_config_and_override():
    cfg = EXL3Config.from_config({"quant_method": "exl3", "bits": 3, "codebook": "mcg",
                                  "scope": "glm53_routed_experts_only", "layer_bits": {"10": 4}})
    assert cfg.bits == 3
    assert cfg.bits_for_prefix("layers.10.mlp.experts") == 4
    assert cfg.bits_for_prefix("layers.5.mlp.experts") == 3
    assert EXL3Config.override_quantization_method({"quant_method": "exl3"}, None) == "exl3"
    assert EXL3Config.override_quantization_method({"quant_method": "fp8"}, None) is None
    dense = EXL3Config.from_config({"quant_method": "exl3", "bits": 4})
    assert dense.scope == "dense_and_moe"


def test_tensor_storage_kinds():
    ts = {
        "model.language_model.layers.3.self_attn.q_a_proj": {"stored_tensors": {
            "model.language_model.layers.3.self_attn.q_a_proj.trellis": {},
            "model.language_model.layers.3.self_attn.q_a_proj.suh": {}}},
        "model.language_model.layers.3.mlp.gate": {"stored_tensors": {
            "model.language_model.layers.3.mlp.gate.weight": {}}},
        "hc_expand": {"stored_tensors": {}},
    }
    kinds = _tensor_storage_kinds(ts)
    assert kinds["model.language_model.layers.3.self_attn.q_a_proj"] == "exl3"
    assert kinds["model.layers.3.self_attn.q_a_proj"] == "exl3"
    assert kinds["model.language_model.layers.3.mlp.gate"] == "native"
    assert "hc_expand" not in kinds
    assert _tensor_storage_kinds(None) == {}


def test_bits_from_trellis_shapes_and_storage_first():
    def tr(shape):
        return {"stored_tensors": {"x.trellis": {"shape": shape}}}
    ts = {
        "model.language_model.layers.3.self_attn.q_b_proj": tr([64, 128, 48]),
        "model.language_model.layers.3.self_attn.o_proj": tr([64, 128, 64]),
        "model.language_model.layers.3.mlp.experts.0.up_proj": tr([256, 128, 48]),
        "model.language_model.layers.3.mlp.experts.7.down_proj": tr([128, 256, 48]),
        "model.language_model.layers.6.mlp.experts.0.up_proj": tr([256, 128, 32]),
    }
    mod, lay = _tensor_storage_bits(ts)
    assert mod["model.layers.3.self_attn.q_b_proj"] == 3 and mod["model.layers.3.self_attn.o_proj"] == 4
    assert lay == {3: 3, 6: 2}
    with pytest.raises(ValueError):
        _tensor_storage_bits({"a.layers.3.mlp.experts.0.up": tr([1, 1, 48]), "a.layers.3.mlp.experts.1.up": tr([1, 1, 32])})
    cfg = EXL3Config.from_config({"quant_method": "exl3", "bits": 2, "codebook": "mul1", "tensor_storage": ts})
    assert cfg.bits_for_prefix("model.layers.3.mlp.experts") == 3
    assert cfg.bits_for_prefix("model.layers.3.self_attn.o_proj") == 4
    assert cfg.bits_for_prefix("model.layers.9.self_attn.q_a_proj") == 2


def test_get_quant_method_routing():
    class FusedMoE(nn.Module):
        pass

    class RowParallelLinear(nn.Module):
        pass

    class VocabParallelEmbedding(nn.Module):
        pass

    cfg = EXL3Config.from_config({"quant_method": "exl3", "bits": 3, "scope": "glm53_routed_experts_only",
                                  "layer_bits": {"4": 2}})
    m = cfg.get_quant_method(FusedMoE(), "model.layers.4.mlp.experts")
    assert isinstance(m, EXL3MoEMethod) and m.bits == 2
    # routed-only scope: dense linears stay unquantized (None without SGLang)
    assert not isinstance(cfg.get_quant_method(RowParallelLinear(), "model.layers.4.self_attn.o_proj"),
                          EXL3LinearMethod)
    dense = EXL3Config.from_config({"quant_method": "exl3", "bits": 4})
    lm = dense.get_quant_method(RowParallelLinear(), "model.layers.1.self_attn.o_proj")
    assert isinstance(lm, EXL3LinearMethod) and lm.bits == 4
    assert dense.get_quant_method(VocabParallelEmbedding(), "model.embed_tokens") is None
    nr = EXL3Config(bits=3, non_routed_exl3={"bits": 5, "modules": ["shared_experts.down_proj"]})
    lm = nr.get_quant_method(RowParallelLinear(), "model.layers.2.mlp.shared_experts.down_proj")
    assert isinstance(lm, EXL3LinearMethod) and lm.bits == 5


# ------------------------------------------------------------ dense markers

def _linear(K=3, mcg=None, mul1=None, in_f=32, out_f=32):
    trellis = torch.zeros(in_f // 16, out_f // 16, 16 * K, dtype=torch.int16)
    m = None if mcg is None else torch.tensor([mcg], dtype=torch.int32)
    u = None if mul1 is None else torch.tensor([mul1], dtype=torch.int32)
    return EXL3DenseLinear(trellis, torch.ones(in_f, dtype=torch.float16), torch.ones(out_f, dtype=torch.float16),
                           m, u)


def test_dense_codebook_markers():
    lin = _linear(mul1=MUL1_MARKER_SIGNED_INT32)
    assert lin.mul1 and not lin.mcg and lin.codebook == 2
    lin = _linear(mcg=MCG_MARKER_SIGNED_INT32)
    assert lin.mcg and not lin.mul1 and lin.codebook == 1
    lin = _linear()
    assert not lin.mcg and not lin.mul1 and lin.codebook == 0  # no marker: 3INST, as exllamav3
    with pytest.raises(ValueError):
        _linear(mcg=MCG_MARKER_SIGNED_INT32, mul1=MUL1_MARKER_SIGNED_INT32)
    assert _linear(K=3).K == 3 and _linear(K=3).in_features == 32


def test_linear_method_create_and_load_on_cpu():
    m = EXL3LinearMethod(EXL3Config(bits=3), bits=3)
    layer = nn.Module()
    m.create_weights(layer, 64, [32, 48], 64, 80, torch.bfloat16)
    assert layer._exl3_lin_n_shards == 2 and hasattr(layer, "exl3_1_trellis") and hasattr(layer, "weight")
    with pytest.raises(ValueError):
        m.create_weights(nn.Module(), 60, [32], 60, 32, torch.float16)
    with pytest.raises(RuntimeError, match="no trellis"):
        m.process_weights_after_loading(layer)
    assert EXL3LinearMethod._shard_index("k") == 1 and EXL3LinearMethod._shard_index(None) == 0


# --------------------------------------------------------------------- MoE

def test_moe_weight_creation():
    m = EXL3MoEMethod(EXL3Config(bits=3), bits=3)
    layer = nn.Module()
    m.create_weights(layer=layer, num_experts=4, hidden_size=4096, intermediate_size_per_partition=2048,
                     params_dtype=torch.float16)
    for name in EXL3MoEMethod._PARAMS:
        assert hasattr(layer, name), name
    assert tuple(layer.w13_trellis.shape) == (4, 2, 256, 128, 48)
    assert tuple(layer.w2_trellis.shape) == (4, 128, 256, 48)


def test_map_topk_to_local():
    ids = torch.tensor([[0, 1], [2, 5]], dtype=torch.long)
    mapped = map_topk_to_local(ids, n_local=4, expert_map=None)
    assert mapped.tolist() == [[0, 1], [2, 4]]
    emap = torch.tensor([-1, 0, 1, -1, 2, 3], dtype=torch.long)  # EP: global -> local
    got = map_topk_to_local(torch.tensor([[0, 1, 4, 9, -2]]), 4, emap)
    assert got.tolist() == [[4, 0, 2, 4, 4]]


def test_tp_sharding_helpers():
    t = torch.arange(4 * 16 * 8 * 2).reshape(4 * 8, 16, 2)  # [in tiles, out tiles, words]
    assert torch.equal(shard_exl3_col(t, "trellis", 1, 2), t[:, 8:16])
    assert torch.equal(shard_exl3_row(t, "trellis", 1, 2), t[16:32])
    assert torch.equal(shard_exl3_row(t, "trellis", 3, 4), t[24:32])
    assert torch.equal(shard_exl3_col(torch.arange(384), "svh", 1, 3), torch.arange(128, 256))
    assert torch.equal(shard_exl3_row(torch.arange(384), "suh", 2, 3), torch.arange(256, 384))
    # the shared vectors stay whole
    assert torch.equal(shard_exl3_col(torch.arange(384), "suh", 1, 3), torch.arange(384))
    assert torch.equal(shard_exl3_row(torch.arange(384), "svh", 1, 3), torch.arange(384))
    with pytest.raises(ValueError, match="not divisible"):
        shard_exl3_col(t, "trellis", 0, 3)
    # inter 768 over tp=8 gives 96 columns (6 tiles): refused at load, not at apply
    with pytest.raises(ValueError, match="multiple of 8"):
        shard_exl3_col(torch.zeros(4, 48, 2), "trellis", 0, 8)
    with pytest.raises(ValueError, match="multiple of 128"):
        shard_exl3_col(torch.zeros(768), "svh", 0, 8)
    with pytest.raises(ValueError, match="multiple of 128"):
        shard_exl3_row(torch.zeros(768), "suh", 0, 8)


def test_loader_packs_experts_and_markers():
    m = EXL3MoEMethod(EXL3Config(bits=2, codebook="mul1"), bits=2)
    layer = nn.Module()
    m.create_weights(layer, num_experts=2, hidden_size=32, intermediate_size_per_partition=32,
                     params_dtype=torch.float16)
    tr = torch.arange(2 * 2 * 32, dtype=torch.int16).reshape(2, 2, 32)
    m._load_exl3(layer.w13_trellis, tr, "experts.w13_trellis", shard_id="w3", expert_id=1)
    assert torch.equal(layer.w13_trellis[1, 1], tr)
    m._load_exl3(layer.w2_mul1, torch.tensor(MUL1_MARKER_SIGNED_INT32), "experts.w2_mul1", shard_id="w2", expert_id=0)
    assert int(layer.w2_mul1[0, 0]) == MUL1_MARKER_SIGNED_INT32
    with pytest.raises(ValueError):
        m._load_exl3(layer.w13_trellis, tr, "experts.w13_trellis", shard_id="w9", expert_id=0)


def _moe_layer(Ks):
    layer = nn.Module()
    layer.w13_trellis = torch.zeros(1)
    layer._exl3_bits = 2
    inners = [{"gate": _linear(Ks[0], mul1=MUL1_MARKER_SIGNED_INT32),
               "up": _linear(Ks[1], mul1=MUL1_MARKER_SIGNED_INT32),
               "down": _linear(Ks[2], mul1=MUL1_MARKER_SIGNED_INT32)} for _ in range(2)]
    return layer, inners


@pytest.mark.parametrize("Ks", [(3, 3, 3), (2, 2, 2), (3, 3, 2)])
def test_fused_state_takes_k_per_projection_from_trellis(Ks):
    layer, inners = _moe_layer(Ks)
    build_exl3_fused_state(layer, inners)
    assert (layer._exl3_k_gate, layer._exl3_k_up, layer._exl3_k_down) == Ks
    assert set(layer._exl3_ptrs) == {f"{w}_{a}" for w in ("gate", "up", "down") for a in ("trellis", "suh", "svh")}


def test_fused_state_mixed_k_in_one_projection_raises():
    layer, inners = _moe_layer((3, 3, 3))
    inners[0]["gate"] = _linear(2, mul1=MUL1_MARKER_SIGNED_INT32)
    with pytest.raises(RuntimeError, match=r"gate has K=\[2, 3\]"):
        build_exl3_fused_state(layer, inners)


def _loop_args():
    return torch.zeros(1, 4), torch.full((1, 2), -1, dtype=torch.long), torch.zeros(1, 2)


def test_python_loop_refuses_under_capture():
    x, ids, w = _loop_args()
    with mock.patch.object(exl3.torch.cuda, "is_current_stream_capturing", return_value=True):
        with pytest.raises(RuntimeError, match="not CUDA-graph capturable"):
            exl3.apply_exl3_python_loop(x, ids, w, [], None, float("inf"))


def test_python_loop_eager_and_cpu_torch():
    x, ids, w = _loop_args()
    with mock.patch.object(exl3.torch.cuda, "is_current_stream_capturing", return_value=False):
        assert tuple(exl3.apply_exl3_python_loop(x, ids, w, [], None, float("inf")).shape) == (1, 4)
    with mock.patch.object(exl3.torch.cuda, "is_current_stream_capturing", side_effect=RuntimeError("no cuda")):
        assert not exl3._cuda_graph_capture_active()
        assert tuple(exl3.apply_exl3_python_loop(x, ids, w, [], None, float("inf")).shape) == (1, 4)


def test_registration_without_sglang():
    import sglang_exl3

    sglang_exl3.register()  # registers the ops; SGLang absent here, so no method registry to check
    assert hasattr(torch.ops.sglang_exl3, "exl3_moe_layer")
