"""EXL3 quantization config and the routed-expert MoE method for SGLang on gfx950.

Public surface of the reference module src/sglang_exl3/exl3.py restricted to
the quantized-matmul path:

* ``EXL3Config`` (exl3.py:1554-1967): bits / codebook / scope, per-layer bits,
  per-module bits and kinds read from ``tensor_storage`` (storage first),
  non-routed EXL3 selections, and the layer -> method routing of
  ``get_quant_method``.
* ``EXL3MoEMethod`` (exl3.py:1987-2314): stacked expert parameters
  (w13_* [E, 2, ...], w2_* [E, ...]), the checkpoint loader with TP sharding,
  codebook detection from the markers, per-expert linears, device pointer
  tables, and ``apply`` for SGLang's dispatcher forms.
* ``map_topk_to_local`` (exl3.py:494-509), ``apply_exl3_experts``
  (exl3.py:1347-1431) and the eager routed loop ``apply_exl3_python_loop``
  (exl3.py:520-576).

The routed experts run in one call of ``torch.ops.sglang_exl3.exl3_moe_layer``
(device-side routing, no host sync, graph-capturable).  Model-family and
deployment specifics of the reference (FP8/MTP delegates, speculative
decoding, server patches) are not part of this path.
"""

from __future__ import annotations

import logging
import os
import re
from typing import Any, Optional

import torch
import torch.nn.functional as F
from torch.nn.parameter import Parameter

from .base import FusedMoEMethodBase, QuantizationConfig, QuantizeMethodBase, set_weight_attrs
from .base import unquantized_linear_method
from .dense import EXL3DenseLinear, EXL3LinearMethod  # noqa: F401  (re-exported)

logger = logging.getLogger("sglang.exl3")

MCG_MULTIPLIER = 0xCBAC1FED
MCG_MARKER_SIGNED_INT32 = -877912083  # 0xCBAC1FED as int32
MUL1_MULTIPLIER = 0x83DCD12D
MUL1_MARKER_SIGNED_INT32 = -2082680531  # 0x83DCD12D as int32
EXL3_SUFFIXES = ("trellis", "suh", "svh", "mcg", "mul1")
SWIGLU_LIMIT_DEFAULT = float("inf")  # no clamp unless the model asks for one
SUPPORTED_BITS = (2, 3, 4, 5, 6)

_LAYER_RE = re.compile(r"(?:^|\.)layers\.(\d+)(?:\.|$)")

# Merged SGLang modules whose checkpoint tensors are stored per child projection.
_MERGED_STORAGE_CHILDREN = {
    "gate_up_proj": ("gate_proj", "up_proj"),
    "fused_qkv_a_proj_with_mqa": ("q_a_proj", "kv_a_proj_with_mqa"),
}


# ------------------------------------------------------------------ helpers

def _both_spellings(name: str):
    """Packs record "model.language_model.layers.N..." where SGLang passes "model.layers.N..."."""
    yield name
    alt = name.replace("model.language_model.", "model.", 1)
    if alt != name:
        yield alt


def _prefix_has_suffix(prefix: str, suffix: str) -> bool:
    return prefix == suffix or prefix.endswith("." + suffix)


def _suffix_from_mapped_name(weight_name: str) -> str:
    tail = weight_name.rsplit(".", 1)[-1]
    suffix = tail.rsplit("_", 1)[-1]
    if suffix not in EXL3_SUFFIXES:
        raise ValueError(f"EXL3 param suffix {suffix!r} (from {tail!r}) not in {EXL3_SUFFIXES}; "
                         f"full mapped name was {weight_name}")
    return suffix


def _stored(entry) -> dict:
    return dict(((entry or {}).get("stored_tensors") or {}))


def _tensor_storage_kinds(tensor_storage: Any) -> dict[str, str]:
    """Module prefix -> "exl3" (a stored .trellis) or "native" (other stored
    tensors); modules without stored tensors are left out."""
    kinds: dict[str, str] = {}
    for module, entry in dict(tensor_storage or {}).items():
        stored = _stored(entry)
        if not stored:
            continue
        kind = "exl3" if any(str(t).endswith(".trellis") for t in stored) else "native"
        for name in _both_spellings(str(module)):
            kinds[name] = kind
    return kinds


def _trellis_shapes(tensor_storage: Any):
    for module, entry in dict(tensor_storage or {}).items():
        for tname, meta in _stored(entry).items():
            if str(tname).endswith(".trellis"):
                yield str(module), list((meta or {}).get("shape") or [])


def _tensor_storage_out_sizes(tensor_storage: Any) -> dict[str, int]:
    """Output width per EXL3 module from its trellis shape [in/16, out/16, 16K]."""
    out: dict[str, int] = {}
    for module, shape in _trellis_shapes(tensor_storage):
        if len(shape) == 3:
            for name in _both_spellings(module):
                out[name] = int(shape[1]) * 16
    return out


def _tensor_storage_bits(tensor_storage: Any) -> tuple[dict[str, int], dict[int, int]]:
    """Per-module bits and per-layer expert bits from the trellis shapes
    (K = last dim / 16).  Experts of one layer must share K (they are stacked);
    a mixed layer raises."""
    module_bits: dict[str, int] = {}
    layer_bits: dict[int, int] = {}
    for module, shape in _trellis_shapes(tensor_storage):
        if not shape:
            continue
        if int(shape[-1]) % 16:
            raise ValueError(f"bad trellis shape for {module}: {shape}")
        bits = int(shape[-1]) // 16
        for name in _both_spellings(module):
            module_bits[name] = bits
        if ".experts." in module:
            m = re.search(r"(?:^|\.)layers\.(\d+)\.", module)
            if m is not None:
                layer = int(m.group(1))
                prev = layer_bits.setdefault(layer, bits)
                if prev != bits:
                    raise ValueError(f"mixed expert bits in layer {layer}: {prev} vs {bits}")
    return module_bits, layer_bits


def storage_kind_for_prefix(kinds: dict[str, str], prefix: str) -> Optional[str]:
    """tensor_storage kind of a module, resolving merged modules through their children."""
    kind = kinds.get(prefix)
    if kind is not None:
        return kind
    leaf = prefix.rsplit(".", 1)[-1]
    children = _MERGED_STORAGE_CHILDREN.get(leaf)
    if not children:
        return None
    parent = prefix[: len(prefix) - len(leaf)]
    child = {kinds.get(parent + c) for c in children} - {None}
    if len(child) > 1:
        raise RuntimeError(f"EXL3 storage: merged module {prefix} has mixed child kinds {sorted(child)}")
    return child.pop() if child else None


def _narrow_tp(t: torch.Tensor, dim: int, rank: int, size: int, align: int) -> torch.Tensor:
    """Slice `rank` of `size` equal shards along `dim`.  Each shard must be a
    multiple of `align` elements: 128 features (8 trellis tiles), because the
    output rotation of every kernel works on whole 128-wide blocks.  The
    reference checks divisibility only (src/sglang_exl3/exl3.py:347-356); an
    unaligned split is refused here at load time instead of failing at apply."""
    if size <= 1:
        return t
    n = int(t.shape[dim])
    if n % size:
        raise ValueError(f"EXL3 TP shard: dim {dim} size {n} is not divisible by tp={size}")
    c = n // size
    if c % align:
        raise ValueError(f"EXL3 TP shard: dim {dim} size {n} over tp={size} gives {c} per rank, not a multiple "
                         f"of {align} ({'trellis tiles' if align == 8 else 'features'}; the 128-wide Hadamard "
                         "blocks cannot be split)")
    return t.narrow(dim, c * rank, c).contiguous()


def shard_exl3_col(loaded: torch.Tensor, suffix: str, tp_rank: int, tp_size: int) -> torch.Tensor:
    """Column-parallel (gate/up): trellis splits on its output-tile dim, svh with it."""
    if suffix == "trellis":
        return _narrow_tp(loaded, 1, tp_rank, tp_size, 8)
    if suffix == "svh":
        return _narrow_tp(loaded, 0, tp_rank, tp_size, 128)
    return loaded.contiguous()


def shard_exl3_row(loaded: torch.Tensor, suffix: str, tp_rank: int, tp_size: int) -> torch.Tensor:
    """Row-parallel (down): trellis splits on its input-tile dim, suh with it."""
    if suffix == "trellis":
        return _narrow_tp(loaded, 0, tp_rank, tp_size, 8)
    if suffix == "suh":
        return _narrow_tp(loaded, 0, tp_rank, tp_size, 128)
    return loaded.contiguous()


def _tp_rank_size() -> tuple[int, int]:
    try:  # pragma: no cover - SGLang distributed present
        from sglang.srt.distributed import get_tp_group  # type: ignore

        g = get_tp_group()
        return int(getattr(g, "rank_in_group", 0)), int(getattr(g, "world_size", 1))
    except Exception:  # noqa: BLE001
        return 0, 1


def make_linear_exl3(trellis, suh, svh, mcg=None, mul1=None, out_dtype=torch.float16) -> EXL3DenseLinear:
    """One expert projection as a dense EXL3 linear (views into the stacked parameters)."""
    del out_dtype
    return EXL3DenseLinear(trellis, suh, svh, mcg, mul1)


# ------------------------------------------------------------------- config

class EXL3Config(QuantizationConfig):
    """SGLang quantization config for EXL3 checkpoints on MI355X (gfx950)."""

    _LAYER_RE = _LAYER_RE

    def __init__(self, bits: int = 4, codebook: str = "mcg", scope: str = "glm53_routed_experts_only",
                 **kwargs: Any) -> None:
        super().__init__()
        self.bits = int(bits)
        self.codebook = str(codebook)
        self.scope = str(scope)
        self.layer_bits = {int(k): int(v) for k, v in dict(kwargs.pop("layer_bits", None) or {}).items()}
        for layer, b in self.layer_bits.items():
            if b not in SUPPORTED_BITS:
                raise ValueError(f"unsupported EXL3 bits={b} for layer {layer}")
        self.non_routed_exl3 = dict(kwargs.pop("non_routed_exl3", None) or {})
        nb = self.non_routed_exl3.get("bits")
        if nb is not None and nb not in SUPPORTED_BITS:
            raise ValueError(f"unsupported non_routed_exl3 bits={nb}")
        if self.non_routed_exl3.get("codebook", "mcg") not in ("mcg", "mul1"):
            raise ValueError(f"unsupported non_routed_exl3 codebook={self.non_routed_exl3.get('codebook')!r}")
        self.raw_config = dict(kwargs)
        self.tensor_storage_kinds: dict[str, str] = {}
        self.tensor_storage_out_sizes: dict[str, int] = {}
        self.tensor_storage_bits: dict[str, int] = {}
        self.storage_layer_bits: dict[int, int] = {}
        self.mtp_bits = self.bits
        self.non_routed_quantization = None
        self.non_routed_dtype_policy = ""
        if self.codebook not in ("mcg", "mul1"):
            raise ValueError(f"unsupported codebook={self.codebook!r}; must be 'mcg' or 'mul1'")
        if self.bits not in SUPPORTED_BITS:
            raise ValueError(f"unsupported EXL3 bits={self.bits}")

    # -- SGLang QuantizationConfig interface
    def get_name(self) -> str:
        return "exl3"

    def get_supported_act_dtypes(self) -> list[torch.dtype]:
        return [torch.bfloat16, torch.float16, torch.float32]

    @classmethod
    def get_min_capability(cls) -> int:
        return 80

    @staticmethod
    def get_config_filenames() -> list[str]:
        return ["quantization_config.json"]

    def get_scaled_act_names(self) -> list[str]:
        return []

    def apply_weight_name_mapper(self, hf_to_sglang_mapper: Any) -> None:
        return None

    @classmethod
    def override_quantization_method(cls, hf_quant_cfg: dict, user_quant: Optional[str], hf_config: Any = None):
        return "exl3" if str((hf_quant_cfg or {}).get("quant_method", "")).lower() == "exl3" else None

    @classmethod
    def from_config(cls, config: dict) -> "EXL3Config":
        skip = {"bits", "codebook", "scope", "quant_method", "tensor_storage", "non_routed_exl3",
                "non_routed_quantization", "mtp_experts", "mtp_experts_start_layer"}
        inst = cls(bits=int(config.get("bits", 4)), codebook=str(config.get("codebook", "mcg")),
                   scope=str(config.get("scope", "glm53_routed_experts_only")),
                   non_routed_exl3=config.get("non_routed_exl3"),
                   **{k: v for k, v in config.items() if k not in skip})
        # a config that only names quant_method=exl3 is a dense pack: every linear is EXL3
        if "scope" not in config and str(config.get("quant_method", "")).lower() == "exl3":
            inst.scope = "dense_and_moe"
        inst.non_routed_quantization = config.get("non_routed_quantization")
        inst.non_routed_dtype_policy = str(config.get("non_routed_dtype_policy", ""))
        inst.mtp_experts = str(config.get("mtp_experts", "exl3"))
        inst.mtp_experts_start_layer = config.get("mtp_experts_start_layer")
        ts = config.get("tensor_storage")
        inst.tensor_storage_kinds = _tensor_storage_kinds(ts)
        inst.tensor_storage_out_sizes = _tensor_storage_out_sizes(ts)
        inst.tensor_storage_bits, inst.storage_layer_bits = _tensor_storage_bits(ts)
        mb = config.get("mtp_bits", config.get("bits", inst.bits))
        inst.mtp_bits = int(mb) if mb is not None else inst.bits
        return inst

    # -- bits per module
    def bits_for_prefix(self, prefix: str) -> int:
        """Stored trellis width first (per module, then per expert layer), then
        the configured per-layer bits, then the default."""
        if prefix in self.tensor_storage_bits:
            return self.tensor_storage_bits[prefix]
        m = _LAYER_RE.search(prefix or "")
        if m is not None and int(m.group(1)) in self.storage_layer_bits:
            return self.storage_layer_bits[int(m.group(1))]
        if m is None or not self.layer_bits:
            return self.bits
        return self.layer_bits.get(int(m.group(1)), self.bits)

    def merged_split_sizes(self, prefix: str) -> Optional[list[int]]:
        """Per-child output widths of a merged module stored as separate EXL3 children."""
        leaf = (prefix or "").rsplit(".", 1)[-1]
        children = _MERGED_STORAGE_CHILDREN.get(leaf)
        if not children:
            return None
        parent = prefix[: len(prefix) - len(leaf)]
        sizes = [self.tensor_storage_out_sizes.get(parent + c) for c in children]
        return None if any(s is None for s in sizes) else [int(s) for s in sizes]

    def _matches_non_routed_exl3(self, prefix: str) -> bool:
        nr = self.non_routed_exl3
        if not nr:
            return False
        if prefix in (nr.get("layers") or {}):
            return True
        return any(_prefix_has_suffix(prefix, m) for m in nr.get("modules", []) or [])

    def _bits_for_non_routed(self, prefix: str) -> int:
        nr = self.non_routed_exl3
        if not nr:
            return self.bits
        layers = nr.get("layers") or {}
        if prefix in layers:
            return int(layers[prefix].get("bits", nr.get("bits", self.bits)))
        for suffix in nr.get("modules", []) or []:
            if _prefix_has_suffix(prefix, suffix):
                per = nr.get("layer_bits") or {}
                if suffix in per:
                    return int(per[suffix])
                break
        return int(nr.get("bits", self.bits))

    # -- routing
    @staticmethod
    def _is_draft(prefix_lower: str) -> bool:
        return "stages." in prefix_lower or "mtp" in prefix_lower or "nextn" in prefix_lower

    def get_quant_method(self, layer: torch.nn.Module, prefix: str) -> Optional[QuantizeMethodBase]:
        cls_name = layer.__class__.__name__
        pl = (prefix or "").lower()
        draft = self._is_draft(pl)
        if ("MoE" in cls_name or "RoutedExperts" in cls_name or hasattr(layer, "num_local_experts")):
            if draft:
                if os.environ.get("SGLANG_EXL3_MTP_EXL3", "1") != "1":
                    return None
                return EXL3MoEMethod(self, bits=int(self.mtp_bits or self.bits_for_prefix(prefix)))
            return EXL3MoEMethod(self, bits=self.bits_for_prefix(prefix))
        if "RadixAttention" in cls_name:
            return None
        is_lm_head = "lm_head" in pl or "ParallelLMHead" in cls_name
        if "VocabParallelEmbedding" in cls_name and not is_lm_head:
            return None
        if not (is_lm_head or "Linear" in cls_name):
            return None
        nr = self.non_routed_exl3 or {}
        if any(_prefix_has_suffix(prefix, m) for m in nr.get("bf16_modules", []) or []):
            return unquantized_linear_method()
        if (not draft and self.tensor_storage_kinds
                and storage_kind_for_prefix(self.tensor_storage_kinds, prefix) != "exl3"):
            return unquantized_linear_method()
        if not draft and (self.scope in ("dense_and_moe", "dense") or os.environ.get("SGLANG_EXL3_DENSE", "0") == "1"):
            method = EXL3LinearMethod(self, bits=self.bits_for_prefix(prefix))
            method.split_sizes = self.merged_split_sizes(prefix)
            return method
        if not draft and self._matches_non_routed_exl3(prefix):
            return EXL3LinearMethod(self, bits=self._bits_for_non_routed(prefix))
        if draft and os.environ.get("SGLANG_EXL3_MTP_EXL3", "1") == "1":
            bits = self._bits_for_non_routed(prefix) if self._matches_non_routed_exl3(prefix) else self.mtp_bits
            return EXL3LinearMethod(self, bits=int(bits))
        return unquantized_linear_method()


# ----------------------------------------------------------------- routing

def pin_exl3_expert_map(layer: torch.nn.Module, device: torch.device) -> Optional[torch.Tensor]:
    emap = getattr(layer, "expert_map", None)
    if emap is None:
        return None
    if emap.device != device or emap.dtype != torch.long:
        layer.expert_map = emap.to(device=device, dtype=torch.long)
    return layer.expert_map


def map_topk_to_local(ids: torch.Tensor, n_local: int, expert_map: Optional[torch.Tensor]) -> torch.Tensor:
    """Global top-k ids -> local expert ids; non-local or invalid ids become
    the sentinel n_local (which every expert kernel skips)."""
    flat = ids.reshape(-1)
    sentinel = flat.new_full(flat.shape, n_local)
    if expert_map is None:
        bad = (flat < 0) | (flat >= n_local)
        return torch.where(bad, sentinel, flat).reshape(ids.shape)
    if expert_map.device != flat.device or expert_map.dtype != torch.long:
        raise RuntimeError("EXL3 expert_map is not pinned to the hidden-state device; "
                           "call pin_exl3_expert_map before fused apply")
    n_global = int(expert_map.numel())
    if n_global == 0:
        return sentinel.reshape(ids.shape)
    mapped = expert_map[flat.clamp(0, n_global - 1)]
    bad = (flat < 0) | (flat >= n_global) | (mapped < 0) | (mapped >= n_local)
    return torch.where(bad, sentinel, mapped).reshape(ids.shape)


def _cuda_graph_capture_active() -> bool:
    try:
        return bool(torch.cuda.is_current_stream_capturing())
    except Exception:  # noqa: BLE001 - CPU-only torch raises here
        return False


def apply_exl3_python_loop(x2d: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor, inners: list,
                           expert_map: Optional[torch.Tensor], limit: float, *, only_experts=None,
                           out: Optional[torch.Tensor] = None, layer=None) -> torch.Tensor:
    """Eager per-expert routed loop (fp32 result): for each expert with tokens,
    gate/up linears, silu(min(g, L)) * clamp(u, -L, L), down linear, weighted
    index_add.  Host-synchronising, so refused under graph capture."""
    del layer
    if _cuda_graph_capture_active():
        raise RuntimeError("EXL3 python-loop MoE is not CUDA-graph capturable (torch.unique/.tolist()/nonzero "
                           "sync the stream); use the fused exl3_moe_layer path under graph capture")
    tokens, hidden = x2d.shape
    if out is None:
        out = torch.zeros(tokens, hidden, dtype=torch.float32, device=x2d.device)
    for raw in torch.unique(ids).tolist():
        e = int(raw)
        if e < 0:
            continue
        if expert_map is not None:
            e = int(expert_map[e].item()) if expert_map.numel() > e else e
            if e < 0:
                continue
        if e >= len(inners) or (only_experts is not None and e not in only_experts):
            continue
        tok, slot = (ids == int(raw)).nonzero(as_tuple=True)
        h = x2d.index_select(0, tok).to(torch.float16).contiguous()
        pack = inners[e]
        g = pack["gate"].forward(h, {}, out_dtype=torch.float32)
        u = pack["up"].forward(h, {}, out_dtype=torch.float32)
        act = F.silu(g.clamp(max=limit)) * u.clamp(min=-limit, max=limit)
        d = pack["down"].forward(act.to(torch.float16).contiguous(), {}, out_dtype=torch.float32)
        out.index_add_(0, tok, d * weights[tok, slot].unsqueeze(-1).to(torch.float32))
    return out


def build_exl3_fused_state(layer: torch.nn.Module, inners: list) -> None:
    """Device pointer tables of the experts' weights (indexed by local id) and
    the per-projection K read from the trellis shapes.  One K per projection
    across the experts (they run in one launch); a mix raises."""
    device = layer.w13_trellis.device

    def table(which: str, attr: str) -> torch.Tensor:
        return torch.tensor([int(getattr(p[which], attr).data_ptr()) for p in inners], dtype=torch.int64,
                            device=device)

    for which in ("gate", "up", "down"):
        ks = sorted({p[which].K for p in inners})
        if len(ks) != 1:
            raise RuntimeError(f"EXL3 fused MoE needs one K per projection; {which} has K={ks}")
        setattr(layer, f"_exl3_k_{which}", ks[0])
    layer._exl3_ptrs = {f"{w}_{a}": table(w, a) for w in ("gate", "up", "down") for a in ("trellis", "suh", "svh")}
    layer._exl3_k = int(getattr(layer, "_exl3_bits", layer._exl3_k_gate))


_TABLE_ORDER = tuple(f"{w}_{a}" for w in ("gate", "up", "down") for a in ("trellis", "suh", "svh"))


def _native_moe_ok(layer, tokens: int, topk: int) -> Optional[str]:
    """Reason the one-call HIP layer cannot run this input, or None."""
    if not isinstance(getattr(layer, "_exl3_ptrs", None), dict):
        return "no pointer tables"
    ks = [getattr(layer, f"_exl3_k_{w}", None) for w in ("gate", "up", "down")]
    if any(not isinstance(k, int) or not 1 <= k <= 8 for k in ks):
        return f"K per projection {ks} outside integer 1..8"
    if layer._exl3_hidden_size % 128 or layer._exl3_intermediate_local % 128:
        return "hidden/intermediate not multiples of 128"
    return None


def apply_exl3_experts(x: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor, layer: torch.nn.Module,
                       *, limit: float = SWIGLU_LIMIT_DEFAULT, fused: Optional[bool] = None) -> torch.Tensor:
    """Routed experts of one MoE layer: [T, hidden] in x's dtype.  Runs the
    one-call HIP layer (device routing, graph-capturable); the eager loop only
    when that path cannot take the input (or fused=False)."""
    inners = getattr(layer, "_exl3_inners", None)
    if not inners:
        raise RuntimeError("EXL3 experts were not built after weight load")
    tokens, hidden = x.shape[-2], x.shape[-1]
    x2d = x.reshape(tokens, hidden)
    ids = topk_ids.reshape(tokens, -1).to(torch.long)
    w = topk_weights.reshape(tokens, -1)
    expert_map = pin_exl3_expert_map(layer, x2d.device)
    local = map_topk_to_local(ids, len(inners), expert_map)
    reason = _native_moe_ok(layer, tokens, int(local.shape[-1]))
    if fused is not False and reason is None:
        lim = float(limit)
        lim = 0.0 if (lim != lim or lim == float("inf")) else lim
        out = torch.ops.sglang_exl3.exl3_moe_layer(
            x2d, local.to(torch.int32), w.to(torch.float32), *[layer._exl3_ptrs[k] for k in _TABLE_ORDER],
            layer._exl3_k_gate, layer._exl3_k_up, layer._exl3_k_down, bool(layer._exl3_use_mcg),
            int(layer._exl3_intermediate_local), lim, int(getattr(layer, "_exl3_codebook", -1)))
        layer._exl3_last_apply = "native"
        return out.to(x.dtype)
    if fused is True:
        raise RuntimeError(f"EXL3 fused MoE requested but unavailable: {reason}")
    layer._exl3_last_apply = "loop"
    return apply_exl3_python_loop(x2d, local, w, inners, None, float(limit)).to(x.dtype)


# --------------------------------------------------------------- MoE method

class EXL3MoEMethod(FusedMoEMethodBase):
    """SGLang fused-MoE method for EXL3 routed experts."""

    _PARAMS = ("w13_trellis", "w13_suh", "w13_svh", "w13_mcg", "w13_mul1",
               "w2_trellis", "w2_suh", "w2_svh", "w2_mcg", "w2_mul1")

    def __init__(self, quant_config: EXL3Config, bits: Optional[int] = None) -> None:
        super().__init__()
        self.quant_config = quant_config
        self.bits = int(bits) if bits is not None else int(quant_config.bits)
        self._logged = False

    def create_weights(self, layer: torch.nn.Module, num_experts: int, hidden_size: int,
                       intermediate_size_per_partition: int, params_dtype: torch.dtype, **extra_weight_attrs) -> None:
        del params_dtype
        inter = intermediate_size_per_partition
        if hidden_size % 16 or inter % 16:
            raise ValueError(f"EXL3 trellis tiles are 16-wide; hidden={hidden_size} intermediate_local={inter}")
        kw = self.bits * 16
        ti, to = hidden_size // 16, inter // 16
        shapes = {
            "w13_trellis": ((num_experts, 2, ti, to, kw), torch.int16),
            "w13_suh": ((num_experts, 2, hidden_size), torch.float16),
            "w13_svh": ((num_experts, 2, inter), torch.float16),
            "w13_mcg": ((num_experts, 2, 1), torch.int32),
            "w13_mul1": ((num_experts, 2, 1), torch.int32),
            "w2_trellis": ((num_experts, to, ti, kw), torch.int16),
            "w2_suh": ((num_experts, inter), torch.float16),
            "w2_svh": ((num_experts, hidden_size), torch.float16),
            "w2_mcg": ((num_experts, 1), torch.int32),
            "w2_mul1": ((num_experts, 1), torch.int32),
        }
        extra = {k: v for k, v in extra_weight_attrs.items() if k != "weight_loader"}
        for name, (shape, dtype) in shapes.items():
            make = torch.zeros if name.endswith(("mcg", "mul1")) else torch.empty
            p = Parameter(make(shape, dtype=dtype), requires_grad=False)
            layer.register_parameter(name, p)
            set_weight_attrs(p, extra)
            p.weight_loader = self._load_exl3
            p._exl3_owner = layer
        layer._exl3_hidden_size = hidden_size
        layer._exl3_intermediate_local = inter
        layer._exl3_k_words = kw
        layer._exl3_bits = self.bits

    def _load_exl3(self, param: Parameter, loaded_weight: torch.Tensor, weight_name: str, shard_id: str = "w1",
                   expert_id: int = 0, return_success: bool = False):
        owner = getattr(param, "_exl3_owner", None)
        if owner is not None and hasattr(owner, "_map_global_expert_id_to_local_expert_id"):
            local = owner._map_global_expert_id_to_local_expert_id(expert_id)
            if local == -1:
                return False if return_success else None
            expert_id = local
        rank, size = _tp_rank_size()
        suffix = _suffix_from_mapped_name(weight_name)
        loaded = loaded_weight.detach().contiguous()
        if shard_id in ("w1", "w3"):
            src = shard_exl3_col(loaded, suffix, rank, size)
            dest = param.data[expert_id, 0 if shard_id == "w1" else 1]
        elif shard_id == "w2":
            src = shard_exl3_row(loaded, suffix, rank, size)
            dest = param.data[expert_id]
        else:
            raise ValueError(f"unknown EXL3 shard_id={shard_id}")
        if suffix in ("mcg", "mul1") and src.numel() == 1 and dest.numel() == 1:
            dest.view(-1)[0] = src.reshape(-1)[0].to(dest.dtype)
        elif tuple(dest.shape) == tuple(src.shape):
            dest.copy_(src)
        elif src.numel() == dest.numel():
            dest.copy_(src.reshape(dest.shape))
        else:
            raise RuntimeError(f"EXL3 load shape mismatch {weight_name} shard={shard_id} expert={expert_id}: "
                               f"dest {tuple(dest.shape)} != loaded {tuple(src.shape)}")
        return True if return_success else None

    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        if not hasattr(layer, "w13_trellis"):
            return
        mcg13, mcg2 = layer.w13_mcg.reshape(-1), layer.w2_mcg.reshape(-1)
        mul13, mul2 = layer.w13_mul1.reshape(-1), layer.w2_mul1.reshape(-1)
        n_mcg = int((mcg13 != 0).sum() + (mcg2 != 0).sum())
        n_mul1 = int((mul13 != 0).sum() + (mul2 != 0).sum())
        cfg_mul1 = str(getattr(self.quant_config, "codebook", "mcg") or "mcg") == "mul1"
        if n_mul1 and not n_mcg:
            use_mul1 = True
        elif n_mcg and not n_mul1:
            use_mul1 = False
        else:
            use_mul1 = cfg_mul1  # both or neither: the config decides
            logger.warning("EXL3 MoE markers mcg=%d mul1=%d; using codebook=%s", n_mcg, n_mul1,
                           "mul1" if use_mul1 else "mcg")
        if use_mul1:
            layer.w13_mul1.fill_(MUL1_MARKER_SIGNED_INT32)
            layer.w2_mul1.fill_(MUL1_MARKER_SIGNED_INT32)
            layer.w13_mcg.zero_()
            layer.w2_mcg.zero_()
        else:
            layer.w13_mcg.fill_(MCG_MARKER_SIGNED_INT32)
            layer.w2_mcg.fill_(MCG_MARKER_SIGNED_INT32)
            layer.w13_mul1.zero_()
            layer.w2_mul1.zero_()
        layer._exl3_use_mul1 = use_mul1
        layer._exl3_codebook = 2 if use_mul1 else 1
        layer._exl3_use_mcg = not use_mul1
        inners = []
        for e in range(int(layer.w13_trellis.shape[0])):
            mk = (lambda mcg, mul1: (None, mul1)) if use_mul1 else (lambda mcg, mul1: (mcg, None))
            inners.append({
                "gate": make_linear_exl3(layer.w13_trellis[e, 0], layer.w13_suh[e, 0], layer.w13_svh[e, 0],
                                         *mk(layer.w13_mcg[e, 0], layer.w13_mul1[e, 0])),
                "up": make_linear_exl3(layer.w13_trellis[e, 1], layer.w13_suh[e, 1], layer.w13_svh[e, 1],
                                       *mk(layer.w13_mcg[e, 1], layer.w13_mul1[e, 1])),
                "down": make_linear_exl3(layer.w2_trellis[e], layer.w2_suh[e], layer.w2_svh[e],
                                         *mk(layer.w2_mcg[e], layer.w2_mul1[e])),
            })
        layer._exl3_inners = inners
        build_exl3_fused_state(layer, inners)
        if not self._logged:
            self._logged = True
            logger.info("EXL3 routed experts engaged: bits=%s experts=%d hidden=%d inter=%d codebook=%s", self.bits,
                        len(inners), layer._exl3_hidden_size, layer._exl3_intermediate_local,
                        "mul1" if use_mul1 else "mcg")

    def apply(self, layer: torch.nn.Module, *args, **kwargs) -> Any:
        """Accepts SGLang's dispatcher output (keyword ``dispatch_output`` or a
        positional object with hidden_states / topk_output), or (x,
        topk_weights, topk_ids) positionally or by keyword."""
        dispatch = kwargs.get("dispatch_output")
        if dispatch is None and args and hasattr(args[0], "hidden_states") and hasattr(args[0], "topk_output"):
            dispatch = args[0]
        if dispatch is not None:
            x = dispatch.hidden_states
            topk = dispatch.topk_output
            if not hasattr(topk, "topk_weights") and hasattr(topk, "to_standard"):
                topk = topk.to_standard()
            if not hasattr(topk, "topk_weights"):
                raise ValueError(f"Unsupported SGLang top-k output format: {type(topk)!r}")
            topk_weights, topk_ids = topk.topk_weights, topk.topk_ids
        elif len(args) >= 3:
            x, topk_weights, topk_ids = args[0], args[1], args[2]
        elif all(k in kwargs for k in ("x", "topk_weights", "topk_ids")):
            x, topk_weights, topk_ids = kwargs["x"], kwargs["topk_weights"], kwargs["topk_ids"]
        else:
            raise ValueError(f"Unrecognized EXL3MoEMethod.apply arguments: args={args}, kwargs={kwargs}")
        limit = getattr(getattr(layer, "moe_runner_config", None), "swiglu_limit", None) or SWIGLU_LIMIT_DEFAULT
        out = apply_exl3_experts(x, topk_ids, topk_weights, layer, limit=float(limit))
        if dispatch is None:
            return out
        try:  # pragma: no cover - SGLang present
            from sglang.srt.layers.moe.token_dispatcher.standard import StandardCombineInput  # type: ignore

            return StandardCombineInput(hidden_states=out)
        except Exception:  # noqa: BLE001
            return (out,)
