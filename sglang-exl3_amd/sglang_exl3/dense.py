"""Dense EXL3 linears on the gfx950 HIP kernels.

``EXL3DenseLinear`` holds one EXL3 weight (trellis int16 [k/16, n/16, 16K],
suh, svh, codebook markers) and runs it through the C ABI: exl3_gemv for up to
64 rows, exl3_gemm above.  ``EXL3LinearMethod`` is the SGLang linear method
(same parameter names, shard handling and apply semantics as the reference's
src/sglang_exl3/dense.py:120-398): one EXL3 weight per output shard, outputs
concatenated, optional bias, optional fp32 per-row input scaling, output in
the layer's dtype.  Two compatible shards (gate/up, k/v) sharing the input run
as one batched launch (exl3_p2b_gemv_batched) instead of the reference's
exllamav3 ``exl3_mgemm``.
"""

from __future__ import annotations

import logging
import math
import os
from typing import Any, Optional

import torch
from torch.nn.parameter import Parameter

from . import _lib
from .base import LinearMethodBase, set_weight_attrs

logger = logging.getLogger("sglang.exl3")

__all__ = ["EXL3DenseLinear", "EXL3LinearMethod", "linear_forward", "_mgemm_two", "_mgemm_pair_compatible"]

# Rows up to which two shards sharing one input run as one batched GEMV launch.
FUSED_PAIR_MAX_ROWS = 64


def _marker_on(t: Optional[torch.Tensor]) -> bool:
    return bool(t is not None and t.numel() > 0 and int(t.reshape(-1)[0]) != 0)


def linear_forward(x2: torch.Tensor, trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor, K: int,
                   codebook: int) -> torch.Tensor:
    """fp16 [rows, n] = x2 (fp16 [rows, k]) @ W for any codebook id, through the
    registered op torch.ops.sglang_exl3.exl3_linear (the C ABI's exl3_gemm: GEMV
    kernels up to 12 rows, 8 from 12288 output columns, 7 from 24576, the MFMA
    GEMM above; shapes checked there), so the call stays one traceable op
    under torch.compile and graph capture."""
    from .ops import register_custom_ops

    register_custom_ops()
    if not x2.is_cuda:
        raise RuntimeError("EXL3 linear requires HIP device tensors")
    return torch.ops.sglang_exl3.exl3_linear(x2, trellis, suh, svh, int(K), int(codebook))


class EXL3DenseLinear:
    """One EXL3 weight plus the metadata the kernels need (reference:
    src/sglang_exl3/dense.py:120-157).  K comes from the trellis shape; the
    codebook from the markers: mcg -> MCG, mul1 -> mul1, neither -> 3INST
    (as exllamav3 selects it); both set is an error."""

    __slots__ = ("trellis", "suh", "svh", "K", "mcg", "mul1", "in_features", "out_features")

    def __init__(self, trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor,
                 mcg: Optional[torch.Tensor] = None, mul1: Optional[torch.Tensor] = None):
        self.trellis = trellis.contiguous()
        self.suh = suh.contiguous()
        self.svh = svh.contiguous()
        self.in_features = int(suh.numel())
        self.out_features = int(svh.numel())
        k = self.trellis.shape[-1] / 16
        self.K = int(k) if float(k).is_integer() else k
        mcg_on, mul1_on = _marker_on(mcg), _marker_on(mul1)
        if mcg_on and mul1_on:
            raise ValueError("EXL3 linear has both mcg and mul1 markers set")
        self.mcg = mcg_on
        self.mul1 = mul1_on

    @property
    def codebook(self) -> int:
        return _lib.codebook_id(self.mcg, self.mul1)

    def forward(self, x: torch.Tensor, params: Optional[dict] = None,
                out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        """y = x @ W for x [..., in_features] (any float dtype); fp16 compute."""
        if not isinstance(self.K, int):
            raise RuntimeError(f"EXL3 linear: fractional K={self.K} packs are not supported by the gfx950 kernels")
        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        if x2.dtype != torch.float16 or not x2.is_contiguous():
            x2 = x2.to(torch.float16).contiguous()
        y = linear_forward(x2, self.trellis, self.suh, self.svh, self.K, self.codebook)
        if out_dtype is not None and y.dtype != out_dtype:
            y = y.to(out_dtype)
        return y.view(*shape[:-1], self.out_features)


def _pair_compatible(a: Optional[EXL3DenseLinear], b: Optional[EXL3DenseLinear]) -> bool:
    return (a is not None and b is not None and isinstance(a.K, int) and a.K == b.K
            and a.in_features == b.in_features and a.out_features == b.out_features
            and a.mcg == b.mcg and a.mul1 == b.mul1 and a.codebook != 0)


def _pair_tables(layer, a: EXL3DenseLinear, b: EXL3DenseLinear, dev: torch.device) -> dict:
    cache = getattr(layer, "_exl3_pair_ptrs", None)
    if cache is None:
        cache = {}
        layer._exl3_pair_ptrs = cache
    key = (id(a), id(b))
    if key not in cache:
        cache[key] = {
            "trellis": torch.tensor([a.trellis.data_ptr(), b.trellis.data_ptr()], dtype=torch.int64, device=dev),
            "suh": torch.tensor([a.suh.data_ptr(), b.suh.data_ptr()], dtype=torch.int64, device=dev),
            "svh": torch.tensor([a.svh.data_ptr(), b.svh.data_ptr()], dtype=torch.int64, device=dev),
            "ids": torch.tensor([0, 1], dtype=torch.int32, device=dev),
        }
    return cache[key]


def fused_pair(layer, x2: torch.Tensor, a: EXL3DenseLinear, b: EXL3DenseLinear,
               x2_b: Optional[torch.Tensor] = None):
    """Both linears in one launch (exl3_p2b_gemv_batched): on the shared fp16
    input x2, or a on x2 and b on x2_b (the batched kernel's per-expert input)."""
    t = _pair_tables(layer, a, b, x2.device)
    xv = x2 if x2_b is None or x2_b is x2 else torch.stack((x2, x2_b), dim=0)
    y = torch.ops.sglang_exl3.p2b_gemv_batched(xv, t["trellis"], t["suh"], t["svh"], t["ids"], a.K, a.mcg,
                                               a.out_features)
    return y[0], y[1]


def _mgemm_pair_compatible(lin0: Optional[EXL3DenseLinear], lin1: Optional[EXL3DenseLinear]) -> bool:
    """Whether two linears run as one batched launch: same K, input and output
    widths and codebook, MCG or mul1 (reference: src/sglang_exl3/dense.py:61-70)."""
    return _pair_compatible(lin0, lin1)


def _mgemm_two(layer, x2: torch.Tensor, lin0: EXL3DenseLinear, lin1: EXL3DenseLinear,
               x2_b: Optional[torch.Tensor] = None):
    """(x2 @ W0, x2_b @ W1) for two EXL3 linears; x2_b None (or x2 itself)
    means both read x2 (reference: src/sglang_exl3/dense.py:89-117, called for
    (q, g) and for (k, v) under a value residual in
    src/sglang_exl3/models/ricursive.py:261-281).  A compatible pair of up to
    FUSED_PAIR_MAX_ROWS rows runs as one batched launch; any other pair
    (different widths, K or codebook, or more rows) as two launches.  The
    outputs are fp16 [rows, out_f] and freshly allocated on every call."""
    if x2.dim() != 2:
        raise ValueError(f"_mgemm_two: x2 must be [rows, in_features], got {tuple(x2.shape)}")
    same = x2_b is None or x2_b is x2
    other = x2 if same else x2_b
    if other.dim() != 2 or other.shape[0] != x2.shape[0] or other.shape[1] != lin1.in_features \
            or x2.shape[1] != lin0.in_features:
        raise ValueError(f"_mgemm_two: inputs {tuple(x2.shape)} / {tuple(other.shape)} do not fit linears of "
                         f"{lin0.in_features} / {lin1.in_features} inputs")

    def f16(t):
        return t if t.dtype == torch.float16 and t.is_contiguous() else t.to(torch.float16).contiguous()

    x2 = f16(x2)
    other = x2 if same else f16(other)
    if x2.shape[0] <= FUSED_PAIR_MAX_ROWS and _pair_compatible(lin0, lin1):
        return fused_pair(layer, x2, lin0, lin1, None if same else other)
    return lin0.forward(x2), lin1.forward(other)


class EXL3LinearMethod(LinearMethodBase):
    """SGLang linear method running dense EXL3 weights on the HIP kernels."""

    def __init__(self, quant_config, bits: Optional[int] = None) -> None:
        super().__init__()
        self.quant_config = quant_config
        self.bits = int(bits) if bits is not None else int(getattr(quant_config, "bits", 4))
        self.split_sizes: Optional[list[int]] = None
        self._logged = False

    # -------------------------------------------------------------- weights
    def create_weights(self, layer, input_size_per_partition: int, output_partition_sizes: list[int],
                       input_size: int, output_size: int, params_dtype: torch.dtype, **extra_weight_attrs) -> None:
        split = self.split_sizes
        if split and len(output_partition_sizes) == 1 and sum(split) == output_partition_sizes[0]:
            output_partition_sizes = [int(v) for v in split]
        for out in output_partition_sizes:
            if input_size_per_partition % 16 or out % 16:
                raise ValueError(f"EXL3 trellis tiles are 16-wide; in={input_size_per_partition} out={out}")
        extra = {k: v for k, v in extra_weight_attrs.items() if k != "weight_loader"}
        layer._exl3_out_dtype = params_dtype or torch.bfloat16
        if not hasattr(layer, "weight"):
            # placeholder some SGLang model code probes for dtype; never loaded or read
            layer.register_parameter("weight", Parameter(torch.empty(0, dtype=torch.int16), requires_grad=False))
        n_shards = len(output_partition_sizes)
        layer._exl3_lin_packs = [dict.fromkeys(("trellis", "suh", "svh", "mcg", "mul1")) for _ in range(n_shards)]
        layer._exl3_lin_n_shards = n_shards
        layer._exl3_lin_input_size_per_partition = int(input_size_per_partition)
        layer._exl3_lin_output_partition_sizes = [int(v) for v in output_partition_sizes]
        layer._exl3_linears = None
        for i in range(n_shards):
            for suffix in ("trellis", "suh", "svh", "mcg", "mul1"):
                p = Parameter(torch.empty(0), requires_grad=False)
                layer.register_parameter(f"exl3_{i}_{suffix}", p)
                set_weight_attrs(p, extra)
                p.weight_loader = self._load_linear
                p._exl3_owner = layer
                p._exl3_shard = i
                p._exl3_suffix = suffix

    @staticmethod
    def _shard_index(shard_id) -> int:
        if shard_id is None:
            return 0
        if isinstance(shard_id, str):
            named = {"q": 0, "k": 1, "v": 2}
            if shard_id in named:
                return named[shard_id]
            try:
                return int(shard_id)
            except ValueError as exc:
                raise ValueError(f"unknown EXL3 linear shard {shard_id!r}") from exc
        return int(shard_id)

    def _load_linear(self, param, loaded_weight: torch.Tensor, shard_id=None) -> None:
        layer = getattr(param, "_exl3_owner", None)
        suffix = getattr(param, "_exl3_suffix", None)
        if layer is None or suffix is None:
            return
        pack = layer._exl3_lin_packs[self._shard_index(shard_id)]
        src = loaded_weight.detach()
        dev = torch.device("cuda", torch.cuda.current_device()) if torch.cuda.is_available() else src.device
        if suffix in ("mcg", "mul1") and src.numel() == 1:
            pack[suffix] = torch.tensor([int(src.reshape(()).item())], dtype=torch.int32, device=dev)
            return
        if suffix in ("suh", "svh"):
            src = src.to(torch.float16)
        pack[suffix] = src.to(device=dev).contiguous()

    def process_weights_after_loading(self, layer) -> None:
        packs = getattr(layer, "_exl3_lin_packs", None)
        if not packs:
            return
        linears = []
        for i, pack in enumerate(packs):
            if pack.get("trellis") is None:
                raise RuntimeError(f"EXL3 linear shard {i} received no trellis tensor; checkpoint/quantization mismatch?")
            if pack.get("suh") is None or pack.get("svh") is None:
                raise RuntimeError(f"EXL3 linear shard {i} missing suh/svh sign vectors")
            linears.append(EXL3DenseLinear(pack["trellis"], pack["suh"], pack["svh"], pack.get("mcg"),
                                           pack.get("mul1")))
        layer._exl3_linears = linears
        if not self._logged:
            self._logged = True
            logger.info("EXL3 dense linears engaged: shards=%d K=%s", len(linears), [lin.K for lin in linears])

    # -------------------------------------------------------------- forward
    def _prepare(self, layer, x: torch.Tensor):
        shape = x.shape
        rows = math.prod(shape[:-1]) if len(shape) > 1 else 1
        scale = None
        if getattr(layer, "_exl3_scale_input", False):
            # fp32 per-row dynamic scaling for inputs that would overflow fp16
            xf = x.reshape(rows, shape[-1]).float()
            scale = (xf.abs().amax(dim=-1, keepdim=True) / 16.0).clamp_min_(1e-6)
            x2 = (xf / scale).to(torch.float16).contiguous()
        else:
            x2 = x.reshape(rows, shape[-1])
            if x2.dtype != torch.float16 or not x2.is_contiguous():
                x2 = x2.to(torch.float16).contiguous()
        return shape, rows, x2, scale

    def apply(self, layer, x: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        linears = getattr(layer, "_exl3_linears", None)
        if not linears:
            raise RuntimeError("EXL3 linear layers were not built after weight load")
        shape, rows, x2, scale = self._prepare(layer, x)
        fuse = rows <= FUSED_PAIR_MAX_ROWS and os.environ.get("SGLANG_EXL3_MGEMM", "1") != "0"
        n = len(linears)
        if n == 2 and fuse and _pair_compatible(linears[0], linears[1]):
            y = torch.cat(fused_pair(layer, x2, linears[0], linears[1]), dim=1)
        elif n == 3 and fuse and _pair_compatible(linears[1], linears[2]):
            q = linears[0].forward(x2)
            k, v = fused_pair(layer, x2, linears[1], linears[2])
            y = torch.cat((q, k, v), dim=1)
        else:
            outs = [lin.forward(x2) for lin in linears]
            y = torch.cat(outs, dim=1) if len(outs) > 1 else outs[0]
        out_dtype = getattr(layer, "_exl3_out_dtype", x.dtype)
        y = (y.float() * scale).to(out_dtype) if scale is not None else y.to(out_dtype)
        if bias is not None:
            y = y + bias.to(out_dtype)
        return y.view(*shape[:-1], y.shape[-1])

    def apply_kv_only(self, layer, x: torch.Tensor):
        """K and V shards of a 3-shard qkv projection only (Q skipped)."""
        linears = getattr(layer, "_exl3_linears", None)
        if not linears or len(linears) != 3:
            raise RuntimeError("apply_kv_only requires a 3-shard qkv_proj")
        shape, rows, x2, _ = self._prepare(layer, x)
        kl, vl = linears[1], linears[2]
        if rows <= FUSED_PAIR_MAX_ROWS and _pair_compatible(kl, vl) and os.environ.get("SGLANG_EXL3_MGEMM", "1") != "0":
            k, v = fused_pair(layer, x2, kl, vl)
        else:
            k, v = kl.forward(x2), vl.forward(x2)
        out_dtype = getattr(layer, "_exl3_out_dtype", x.dtype)
        k, v = k.to(out_dtype), v.to(out_dtype)
        return k.view(*shape[:-1], k.shape[-1]), v.view(*shape[:-1], v.shape[-1])
