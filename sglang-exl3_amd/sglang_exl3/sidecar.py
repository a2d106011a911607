"""Checkpoint EXL3 groups -> the per-shard parameters of dense EXL3 linears.

Reference behaviour: src/sglang_exl3/sidecar.py:1-120 (same public names,
same routing outcomes).  The code here is organised around one resolution
step and one delivery step:

* ``resolve(params, name)`` turns a checkpoint name into a ``Destination``
  (layer module, group member, shard index or "cut over every shard"), or
  None when the name is not a dense EXL3 group member of a layer that
  ``params`` holds.  It takes two table lookups: the name's last component
  must be an EXL3 group member (``SIDECAR_SUFFIXES``), and the module leaf
  may be one SGLang merges into a wider layer (``MERGED_LEAVES``).  The
  layer's shard count is read from the parameter names
  ``EXL3LinearMethod`` registers, ``<layer>.exl3_<i>_<member>``.
* ``deliver(params, dest, tensor)`` hands the tensor (or, for a fused
  group, its per-shard views from ``split_fused_group``) to the shard
  parameters' ``weight_loader``.

``split_fused_group`` is driven by ``OUTPUT_AXIS``: per member, the tensor
dimension that runs along the output features and how many output features
one index along it covers (trellis: 16-wide tiles in dimension 1; svh: one
feature per element).  Members without an output axis (suh runs along the
input features; mcg / mul1 are scalar markers) go to every shard whole.

A name that resolves to nothing returns False from ``route_exl3_sidecar``,
so a caller that checks every shard received a trellis fails closed.
"""

from __future__ import annotations

from dataclasses import dataclass
from itertools import accumulate, count
from typing import Any, Dict, List, Optional, Tuple

import torch

# Members of one EXL3 checkpoint group (the checkpoint format's names).
SIDECAR_SUFFIXES = ("trellis", "suh", "svh", "mcg", "mul1")
TILE = 16

# Checkpoint module leaf -> (leaf of the SGLang layer it is merged into, shard
# index in that layer).  The names are SGLang's merged-layer names.
MERGED_LEAVES = {
    "q_a_proj": ("fused_qkv_a_proj_with_mqa", 0),
    "kv_a_proj_with_mqa": ("fused_qkv_a_proj_with_mqa", 1),
    "gate_proj": ("gate_up_proj", 0),
    "up_proj": ("gate_up_proj", 1),
}

# Layer leaves whose checkpoint group may hold all shards fused along the
# output axis (q | k | v).
FUSED_LEAVES = frozenset({"qkv_proj"})

# Group member -> (dimension along the output features, output features per
# index along it, tensor rank).
OUTPUT_AXIS = {"trellis": (1, TILE, 3), "svh": (0, 1, 1)}


@dataclass(frozen=True)
class Destination:
    """Where one checkpoint group member goes: parameter
    ``<layer>.exl3_<shard>_<member>``, or every shard of ``layer`` (cut along
    the output axis) when ``shard`` is None."""

    layer: str
    member: str
    shard: Optional[int]
    shards: int

    def key(self, shard: int) -> str:
        return f"{self.layer}.exl3_{shard}_{self.member}"


def split_sidecar_name(name: str) -> Optional[Tuple[str, str]]:
    """``"a.b.trellis"`` -> ``("a.b", "trellis")``; None for a name whose last
    component is not an EXL3 group member, or that has no module part."""
    module, sep, member = name.rpartition(".")
    return (module, member) if sep and module and member in SIDECAR_SUFFIXES else None


def shard_count(params: Dict[str, Any], layer: str) -> int:
    """Shards 0, 1, ... that ``layer`` registered (0: not a dense EXL3 layer)."""
    return next(i for i in count() if f"{layer}.exl3_{i}_trellis" not in params)


def split_fused_group(owner_sizes: List[int], suffix: str, tensor: torch.Tensor) -> List[torch.Tensor]:
    """Per-shard views of a group stored fused along the output axis.

    ``owner_sizes``: output features of each shard (positive multiples of 16,
    summing to the group's width).  Members with an output axis
    (``OUTPUT_AXIS``) are cut along it with ``torch.split``; the others are
    returned whole, once per shard."""
    widths = [int(s) for s in owner_sizes]
    bad = [w for w in widths if w <= 0 or w % TILE]
    if bad:
        raise ValueError(f"EXL3 fused group: shard widths {widths} must be positive multiples of {TILE} ({bad})")
    axis = OUTPUT_AXIS.get(suffix)
    if axis is None:
        return [tensor] * len(widths)
    dim, per_index, rank = axis
    total = list(accumulate(widths))[-1]
    if tensor.dim() != rank or int(tensor.shape[dim]) * per_index != total:
        raise ValueError(f"EXL3 fused group: {suffix} of shape {tuple(tensor.shape)} cannot be cut into "
                         f"output widths {widths} (total {total})")
    return list(torch.split(tensor, [w // per_index for w in widths], dim=dim))


def resolve(params: Dict[str, Any], name: str) -> Optional[Destination]:
    """The Destination of checkpoint tensor ``name``, or None when it is not a
    dense EXL3 group member here (not a group member name, a routed expert's
    group, a name the model owns itself, or a module without EXL3 shards)."""
    parsed = split_sidecar_name(name)
    if parsed is None or name in params or ".experts." in name:
        return None
    module, member = parsed
    parent, _, leaf = module.rpartition(".")
    merged = MERGED_LEAVES.get(leaf)
    layer = module if merged is None else (f"{parent}.{merged[0]}" if parent else merged[0])
    shard = 0 if merged is None else merged[1]
    shards = shard_count(params, layer)
    if shards == 0:
        return None
    if leaf in FUSED_LEAVES and shards > 1:
        return Destination(layer, member, None, shards)
    if shard >= shards:
        raise RuntimeError(f"EXL3 checkpoint tensor {name} belongs to shard {shard} of {layer}, "
                           f"which registered {shards} shard(s)")
    return Destination(layer, member, shard, shards)


def deliver(params: Dict[str, Any], dest: Destination, tensor: torch.Tensor) -> None:
    """Hand ``tensor`` to the shard parameter(s) ``dest`` names through their
    ``weight_loader``; a fused group is cut at the layer's output partition
    sizes first."""
    if dest.shard is not None:
        p = params[dest.key(dest.shard)]
        p.weight_loader(p, tensor, shard_id=dest.shard)
        return
    owner = params[dest.key(0)]._exl3_owner
    widths = list(owner._exl3_lin_output_partition_sizes)
    if len(widths) != dest.shards:
        raise RuntimeError(f"EXL3 fused group of {dest.layer}: the layer has {dest.shards} shards but "
                           f"output partition sizes {widths}")
    for i, part in enumerate(split_fused_group(widths, dest.member, tensor)):
        p = params[dest.key(i)]
        p.weight_loader(p, part, shard_id=i)


def route_exl3_sidecar(params: Dict[str, Any], name: str, tensor: torch.Tensor) -> bool:
    """Load checkpoint tensor ``name`` into the dense EXL3 shard parameter(s)
    it belongs to.  True: consumed (the caller skips the name); False: not a
    dense EXL3 group member here (reference: src/sglang_exl3/sidecar.py:93-120)."""
    dest = resolve(params, name)
    if dest is None:
        return False
    deliver(params, dest, tensor)
    return True
