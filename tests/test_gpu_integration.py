"""End-to-end GPU checks of the SGLang integration layer: EXL3LinearMethod and
EXL3MoEMethod built through create_weights -> checkpoint loaders ->
process_weights_after_loading -> apply, against the CPU oracle (bar:
max-abs-err <= 2e-2 * rms(ref), cosine >= 0.9999)."""

import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle
from gpu_util import check_close, make_weight, make_x
from sglang_exl3 import ops
from sglang_exl3.exl3 import (
    MCG_MARKER_SIGNED_INT32,
    MUL1_MARKER_SIGNED_INT32,
    EXL3Config,
    EXL3MoEMethod,
    apply_exl3_experts,
)
from sglang_exl3.dense import EXL3DenseLinear, EXL3LinearMethod

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _registered():
    ops.register_custom_ops()


def _scaled(k, n, K, seed):
    tr, su, sv = make_weight(k, n, K, seed)
    return tr, su, (sv.astype(np.float32) * (4.0 / np.sqrt(k))).astype(np.float16)


@pytest.mark.parametrize("rows,shards,marker,cb,dtype", [
    (3, 2, "mcg", 1, torch.float16), (3, 3, "mul1", 2, torch.float16), (80, 2, "mcg", 1, torch.float16),
    (5, 1, None, 0, torch.float16), (1, 2, "mul1", 2, torch.float16), (80, 2, "mcg", 1, torch.bfloat16),
])
def test_linear_method_end_to_end(rows, shards, marker, cb, dtype):
    """fp16 layers are held to the bar; a bf16 layer's output is compared with
    the reference rounded to bf16 (its own rounding exceeds the bar at |y| ~ 20)."""
    print(f"case: linear rows={rows} shards={shards} cb={cb} {dtype}", flush=True)
    k, K = 256, 3
    outs = [256, 128, 128][:shards] if shards == 3 else [256] * shards
    method = EXL3LinearMethod(EXL3Config(bits=K, codebook="mul1" if marker == "mul1" else "mcg"), bits=K)
    layer = nn.Module()
    method.create_weights(layer, k, outs, k, sum(outs), dtype)
    weights = []
    for i, n in enumerate(outs):
        tr, su, sv = _scaled(k, n, K, seed=100 * rows + i)
        weights.append((tr, su, sv))
        p = lambda s: getattr(layer, f"exl3_{i}_{s}")
        method._load_linear(p("trellis"), torch.from_numpy(tr), i)
        method._load_linear(p("suh"), torch.from_numpy(su), i)
        method._load_linear(p("svh"), torch.from_numpy(sv), i)
        if marker:
            val = MCG_MARKER_SIGNED_INT32 if marker == "mcg" else MUL1_MARKER_SIGNED_INT32
            method._load_linear(p(marker), torch.tensor(val, dtype=torch.int32), i)
    method.process_weights_after_loading(layer)
    assert all(lin.codebook == cb for lin in layer._exl3_linears)
    x = make_x(rows, k, seed=rows)
    bias = np.random.default_rng(1).standard_normal(sum(outs)).astype(np.float32)
    y = method.apply(layer, torch.from_numpy(x).cuda().to(dtype).view(1, rows, k), torch.from_numpy(bias).cuda())
    torch.cuda.synchronize()
    assert y.shape == (1, rows, sum(outs)) and y.dtype == dtype
    x16 = torch.from_numpy(x).to(dtype).to(torch.float16).numpy()  # the input the layer saw, as fp16
    ref = np.concatenate([oracle.matmul(x16, oracle.dequant(tr, su, sv, K, cb, rtz=True)) for tr, su, sv in weights],
                         axis=1) + bias
    got = y.float().cpu().numpy().reshape(rows, -1)
    if dtype == torch.bfloat16:
        # bar + one bf16 ulp per element (output rounding of values near a boundary)
        ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - 7)
        rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
        assert np.all(np.abs(got - ref) <= 2e-2 * rms + ulp)
        cos = float(np.dot(got.ravel(), ref.ravel()) / (np.linalg.norm(got) * np.linalg.norm(ref)))
        assert cos >= 0.9999
        return
    check_close(got, ref, f"linear method rows={rows}")


def _build_moe(E, hidden, inter, K, marker, seed):
    cfg = EXL3Config(bits=K, codebook=marker)
    method = EXL3MoEMethod(cfg, bits=K)
    layer = nn.Module()
    method.create_weights(layer, num_experts=E, hidden_size=hidden, intermediate_size_per_partition=inter,
                          params_dtype=torch.float16)
    layer.cuda()
    val = MCG_MARKER_SIGNED_INT32 if marker == "mcg" else MUL1_MARKER_SIGNED_INT32
    cb = 1 if marker == "mcg" else 2
    experts = []
    for e in range(E):
        spec = {}
        for j, (proj, shard, k, n) in enumerate((("gate", "w1", hidden, inter), ("up", "w3", hidden, inter),
                                                  ("down", "w2", inter, hidden))):
            tr, su, sv = _scaled(k, n, K, seed * 1000 + 3 * e + j)
            spec[proj] = (tr, su, sv, K, cb)
            pfx = "w13" if shard != "w2" else "w2"
            for suffix, arr in (("trellis", tr), ("suh", su), ("svh", sv)):
                method._load_exl3(getattr(layer, f"{pfx}_{suffix}"), torch.from_numpy(arr).cuda(),
                                  f"experts.{pfx}_{suffix}", shard_id=shard, expert_id=e)
            method._load_exl3(getattr(layer, f"{pfx}_{marker}"), torch.tensor(val, dtype=torch.int32),
                              f"experts.{pfx}_{marker}", shard_id=shard, expert_id=e)
        experts.append(spec)
    method.process_weights_after_loading(layer)
    return method, layer, experts


@pytest.mark.parametrize("T,topk,E,marker", [(1, 4, 8, "mcg"), (6, 2, 8, "mul1"), (20, 4, 16, "mcg")])
def test_moe_method_end_to_end(T, topk, E, marker):
    print(f"case: moe method T={T} topk={topk} E={E} {marker}", flush=True)
    hidden, inter, K = 256, 256, 3
    method, layer, experts = _build_moe(E, hidden, inter, K, marker, seed=T)
    rng = np.random.default_rng(T)
    ids = np.stack([rng.choice(E, topk, replace=False) for _ in range(T)]).astype(np.int64)
    w = rng.random((T, topk)).astype(np.float32)
    x = make_x(T, hidden, seed=T + 3)
    out = method.apply(layer, torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(), torch.from_numpy(ids).cuda())
    torch.cuda.synchronize()
    assert layer._exl3_last_apply == "native"
    ref = oracle.moe_ref(x, ids, w, experts)
    check_close(out.float().cpu().numpy(), ref, "moe method native")
    # the eager per-expert loop over the same linears agrees too
    loop = apply_exl3_experts(torch.from_numpy(x).cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda(),
                              layer, fused=False)
    torch.cuda.synchronize()
    assert layer._exl3_last_apply == "loop"
    check_close(loop.float().cpu().numpy(), ref, "moe method loop")


def test_moe_method_expert_parallel_map():
    """Global ids mapped through expert_map; ids of other ranks are skipped."""
    E_local, hidden, inter, K = 4, 256, 128, 2
    method, layer, experts = _build_moe(E_local, hidden, inter, K, "mcg", seed=77)
    # 8 global experts, this rank owns globals 4..7 as locals 0..3
    layer.expert_map = torch.tensor([-1, -1, -1, -1, 0, 1, 2, 3], dtype=torch.long)
    ids = np.array([[4, 1], [7, 5], [0, 2]], dtype=np.int64)
    w = np.array([[0.5, 0.5], [0.25, 0.75], [1.0, 1.0]], dtype=np.float32)
    x = make_x(3, hidden, seed=9)
    out = method.apply(layer, torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(), torch.from_numpy(ids).cuda())
    torch.cuda.synchronize()
    local = np.where(ids >= 4, ids - 4, -1)
    ref = oracle.moe_ref(x, local, w, experts)
    o = out.float().cpu().numpy()
    assert np.all(o[2] == 0.0)
    check_close(o, ref, "moe expert map")


def test_dense_linear_forward_3inst():
    tr, su, sv = _scaled(256, 256, 4, seed=5)
    lin = EXL3DenseLinear(torch.from_numpy(tr).cuda(), torch.from_numpy(su).cuda(), torch.from_numpy(sv).cuda())
    x = make_x(2, 256, seed=2)
    y = lin.forward(torch.from_numpy(x).cuda(), {}, out_dtype=torch.float32)
    torch.cuda.synchronize()
    check_close(y.cpu().numpy(), oracle.matmul(x, oracle.dequant(tr, su, sv, 4, 0, rtz=True)), "3inst linear")


def test_moe_method_prefill_batch_stays_native():
    """A 2048-token top-8 batch (16384 routed rows) runs the device-side prefill
    pipeline through EXL3MoEMethod.apply, never the host-synced loop."""
    T, topk, E, hidden, inter, K = 2048, 8, 16, 256, 128, 3
    method, layer, experts = _build_moe(E, hidden, inter, K, "mul1", seed=99)
    rng = np.random.default_rng(98)
    ids = np.stack([rng.choice(E, topk, replace=False) for _ in range(T)]).astype(np.int64)
    w = rng.random((T, topk)).astype(np.float32)
    x = make_x(T, hidden, seed=97)
    out = method.apply(layer, torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(), torch.from_numpy(ids).cuda())
    torch.cuda.synchronize()
    assert layer._exl3_last_apply == "native"
    sel = np.sort(rng.choice(T, 48, replace=False))
    check_close(out.float().cpu().numpy()[sel], oracle.moe_ref(x[sel], ids[sel], w[sel], experts), "moe prefill method")


@pytest.mark.parametrize("rows", [1, 5, 80])
def test_checkpoint_to_forward(tmp_path, rows):
    """A two-shard safetensors checkpoint streamed (iter_safetensors_pread) and routed
    (route_exl3_sidecar: fused qkv group cut into q/k/v shards, gate/up merged) into
    EXL3LinearMethod layers on the device; each layer's apply() against the oracle on the
    checkpoint's own groups."""
    from test_loader_sidecar import build_checkpoint, load_layers

    files, groups, dims = build_checkpoint(tmp_path)
    layers, leftovers = load_layers(files, dims)
    assert leftovers == ["model.norm.weight"]
    cfg = EXL3Config.from_config({"bits": 3, "codebook": "mcg"})

    def ref(x, mods):
        outs = []
        for mod in mods:
            t, su, sv = (a.numpy() for a in groups[mod])
            outs.append(oracle.matmul(x, oracle.dequant(t.view(np.int16), su, sv, 3, 1, rtz=True)))
        return np.concatenate(outs, axis=1)

    cases = {
        "model.layers.0.self_attn.qkv_proj": ["model.layers.0.self_attn.qkv_proj"],
        "model.layers.0.self_attn.o_proj": ["model.layers.0.self_attn.o_proj"],
        "model.layers.0.mlp.gate_up_proj": ["model.layers.0.mlp.gate_proj", "model.layers.0.mlp.up_proj"],
    }
    for prefix, mods in cases.items():
        layer = layers[prefix]
        method = EXL3LinearMethod(cfg, bits=3)
        method.process_weights_after_loading(layer)
        assert all(lin.trellis.is_cuda for lin in layer._exl3_linears)
        k = layer._exl3_lin_input_size_per_partition
        x = make_x(rows, k, seed=rows + len(prefix))
        y = method.apply(layer, torch.from_numpy(x).cuda().to(torch.bfloat16))
        torch.cuda.synchronize()
        assert y.dtype == torch.float16  # the layer's params dtype
        xr = torch.from_numpy(x).to(torch.bfloat16).to(torch.float16).numpy()
        check_close(y.float().cpu().numpy(), ref(xr, mods), f"checkpoint {prefix} rows={rows}")


@pytest.mark.parametrize("rows,n0,n1,K0,K1,cb0,cb1,second", [
    (1, 256, 256, 3, 3, 1, 1, False),     # (q, g): one batched launch on a shared input
    (4, 384, 384, 4, 4, 2, 2, True),      # (k, v) with a value residual: per-linear inputs, one launch
    (8, 256, 128, 3, 3, 1, 1, True),      # unequal widths: two launches
    (2, 256, 256, 3, 2, 1, 1, False),     # different K: two launches
    (3, 256, 256, 3, 3, 1, 2, True),      # different codebooks: two launches
    (80, 256, 256, 3, 3, 2, 2, True),     # above the batched row limit: two launches
])
def test_mgemm_two(rows, n0, n1, K0, K1, cb0, cb1, second):
    """_mgemm_two (reference dense.py:89-117): (x @ W0, x_b @ W1) against the oracle."""
    from sglang_exl3.dense import _mgemm_pair_compatible, _mgemm_two

    k = 256
    w0, w1 = _scaled(k, n0, K0, seed=40 + rows), _scaled(k, n1, K1, seed=41 + rows)
    mk = {1: torch.tensor([1], dtype=torch.int32), 2: None}
    mu = {1: None, 2: torch.tensor([1], dtype=torch.int32)}
    lins = [EXL3DenseLinear(*(torch.from_numpy(a).cuda() for a in w), mcg=mk[cb], mul1=mu[cb])
            for w, cb in ((w0, cb0), (w1, cb1))]
    assert _mgemm_pair_compatible(*lins) == (n0 == n1 and K0 == K1 and cb0 == cb1)
    x = make_x(rows, k, seed=50 + rows)
    xb = make_x(rows, k, seed=60 + rows) if second else None
    layer = nn.Module()
    y0, y1 = _mgemm_two(layer, torch.from_numpy(x).cuda(), *lins,
                        x2_b=None if xb is None else torch.from_numpy(xb).cuda())
    torch.cuda.synchronize()
    assert y0.shape == (rows, n0) and y1.shape == (rows, n1) and y0.dtype == y1.dtype == torch.float16
    ref0 = oracle.matmul(x, oracle.dequant(*w0, K0, cb0, rtz=True))
    ref1 = oracle.matmul(x if xb is None else xb, oracle.dequant(*w1, K1, cb1, rtz=True))
    check_close(y0.float().cpu().numpy(), ref0, f"mgemm first rows={rows}")
    check_close(y1.float().cpu().numpy(), ref1, f"mgemm second rows={rows}")
    # fresh outputs on every call
    z0, _ = _mgemm_two(layer, torch.from_numpy(x).cuda(), *lins,
                       x2_b=None if xb is None else torch.from_numpy(xb).cuda())
    assert z0.data_ptr() != y0.data_ptr() and torch.equal(z0, y0)
