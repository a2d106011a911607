"""Routing of EXL3 checkpoint groups onto the per-shard parameters of dense
EXL3 linears (reference: src/sglang_exl3/sidecar.py:1-120).

A checkpoint stores one group per module: ``<module>.trellis``, ``.suh``,
``.svh`` and the codebook markers ``.mcg`` / ``.mul1``.  ``EXL3LinearMethod``
registers one parameter set ``exl3_{i}_{suffix}`` per output shard of a layer,
so SGLang's stacked-parameter mapping does not know the checkpoint names; this
module maps them:

- ``q_a_proj`` / ``kv_a_proj_with_mqa`` -> shards 0 / 1 of ``fused_qkv_a_proj_with_mqa``;
- ``gate_proj`` / ``up_proj`` -> shards 0 / 1 of ``gate_up_proj``;
- a ``qkv_proj`` stored as ONE group (q|k|v along the output axis) -> cut along
  the 16-wide output tiles into the layer's shards, at the layer's
  ``_exl3_lin_output_partition_sizes``;
- any other EXL3 module -> shard 0.

A name that is not consumed returns False, so the caller's post-load check
(every shard got a trellis) fails closed.
"""

from __future__ import annotations

from typing import Any, Dict, List, Optional, Tuple

import torch

SIDECAR_SUFFIXES = ("trellis", "suh", "svh", "mcg", "mul1")
TILE = 16

# checkpoint module leaf -> (leaf of the merged layer, shard index)
MERGED_LEAVES = {
    "q_a_proj": ("fused_qkv_a_proj_with_mqa", 0),
    "kv_a_proj_with_mqa": ("fused_qkv_a_proj_with_mqa", 1),
    "gate_proj": ("gate_up_proj", 0),
    "up_proj": ("gate_up_proj", 1),
}


def split_sidecar_name(name: str) -> Optional[Tuple[str, str]]:
    """``"a.b.trellis"`` -> ``("a.b", "trellis")``; None for any other name."""
    base, dot, suffix = name.rpartition(".")
    if dot and base and suffix in SIDECAR_SUFFIXES:
        return base, suffix
    return None


def _shard_count(params: Dict[str, Any], module: str) -> int:
    n = 0
    while f"{module}.exl3_{n}_trellis" in params:
        n += 1
    return n


def split_fused_group(owner_sizes: List[int], suffix: str, tensor: torch.Tensor) -> List[torch.Tensor]:
    """Cut one fused group along the output axis into per-shard groups (views).

    ``trellis`` is [in/16, out/16, 16 K] and is cut along its tile columns;
    ``svh`` is [out]; ``suh`` (input axis) and the markers go to every shard
    unchanged.  Every size must be a multiple of 16 and they must sum to the
    group's output width (reference: src/sglang_exl3/sidecar.py:59-90).
    """
    sizes = [int(s) for s in owner_sizes]
    if any(s <= 0 or s % TILE for s in sizes):
        raise ValueError(f"EXL3 fused split: output sizes {sizes} are not positive multiples of {TILE}")
    out = sum(sizes)
    bounds = [0]
    for s in sizes:
        bounds.append(bounds[-1] + s)
    if suffix == "trellis":
        if tensor.dim() != 3 or tensor.shape[1] * TILE != out:
            raise ValueError(f"EXL3 fused trellis of shape {tuple(tensor.shape)} does not hold {out} outputs")
        return [tensor[:, a // TILE:b // TILE, :] for a, b in zip(bounds[:-1], bounds[1:])]
    if suffix == "svh":
        if tensor.dim() != 1 or tensor.shape[0] != out:
            raise ValueError(f"EXL3 fused svh of shape {tuple(tensor.shape)} does not hold {out} outputs")
        return [tensor[a:b] for a, b in zip(bounds[:-1], bounds[1:])]
    return [tensor] * len(sizes)


def route_exl3_sidecar(params: Dict[str, Any], name: str, tensor: torch.Tensor) -> bool:
    """Hand one checkpoint tensor to the EXL3 shard parameter(s) it belongs to.

    True: the tensor was consumed (the caller skips the name).  False: not a
    dense EXL3 group here - not a sidecar name, an expert's group (those go
    through the expert mapping), a name the model owns directly, or a module
    without EXL3 shards (reference: src/sglang_exl3/sidecar.py:93-120).
    """
    parsed = split_sidecar_name(name)
    if parsed is None or ".experts." in name or name in params:
        return False
    module, suffix = parsed
    parent, _, leaf = module.rpartition(".")
    target, shard = module, 0
    if leaf in MERGED_LEAVES:
        merged, shard = MERGED_LEAVES[leaf]
        target = f"{parent}.{merged}" if parent else merged
    n = _shard_count(params, target)
    if n == 0:
        return False
    if leaf == "qkv_proj" and n > 1:
        owner = params[f"{target}.exl3_0_{suffix}"]._exl3_owner
        sizes = list(owner._exl3_lin_output_partition_sizes)
        if len(sizes) != n:
            raise RuntimeError(f"EXL3 fused qkv {target}: {n} shards but output sizes {sizes}")
        for i, part in enumerate(split_fused_group(sizes, suffix, tensor)):
            p = params[f"{target}.exl3_{i}_{suffix}"]
            p.weight_loader(p, part, shard_id=i)
        return True
    if shard >= n:
        raise RuntimeError(f"EXL3 group {name}: shard {shard} but {target} has {n} shard(s)")
    p = params[f"{target}.exl3_{shard}_{suffix}"]
    p.weight_loader(p, tensor, shard_id=shard)
    return True
