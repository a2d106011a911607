"""torch.library custom ops ``torch.ops.sglang_exl3.*`` backed by the gfx950 HIP library.

Same op names, schemas, mutation annotations and fake (meta) kernels as the
reference registry (src/sglang_exl3/ops.py:29-230), so SGLang's graph runner,
piecewise graphs and torch.compile see the same surface.  Every op enqueues
its kernels on the current HIP stream of the input's device through the C
ABI (include/sglang_exl3_amd.h); non-zero statuses become RuntimeError.
CPU tensors are rejected: there is no CPU fallback in the product.
"""

from __future__ import annotations

import logging
from typing import Dict, Tuple

import torch

from . import _lib

logger = logging.getLogger("sglang.exl3.ops")

_OPS_REGISTERED = False

# Reference op list (tests/test_cuda_graph.py:15-23)
OP_NAMES = (
    "dequant_trellis",
    "exl3_gemv",
    "exl3_gemm",
    "p2b_gemv_batched",
    "p2b_fused_moe",
    "exl3_fat_gemm",
    "exl3_fat_gemm_scatter",
)

# ---------------------------------------------------------------- plumbing

_WORKSPACES: Dict[Tuple[int, int], torch.Tensor] = {}
# Buffers some HIP graph was captured with (by id; the dict keeps them alive,
# so an id cannot be reused while it is listed).  A replay writes counters
# and partial sums into the captured addresses, so such a buffer is kept when
# a larger one replaces it (in _RETIRED_WORKSPACES, with its (device, stream)
# key); a replaced buffer that no graph captured is dropped and freed
# (stream-ordered, on the stream it was used on).
_CAPTURED: Dict[int, torch.Tensor] = {}
_RETIRED_WORKSPACES: list = []


def _stream_ptr(t: torch.Tensor) -> int:
    return int(torch.cuda.current_stream(t.device).cuda_stream)


def _require_device(name: str, *tensors: torch.Tensor) -> None:
    for t in tensors:
        if not t.is_cuda:
            raise RuntimeError(f"sglang_exl3::{name} requires HIP device tensors (got {t.device})")
    dev = tensors[0].device
    for t in tensors[1:]:
        if t.device != dev:
            raise RuntimeError(f"sglang_exl3::{name}: tensors on different devices ({dev}, {t.device})")


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Zero-initialised scratch keyed by (device, current stream).  Kernels
    leave their counters zero after each call, so the buffer is reused as is;
    growth allocates a new zeroed buffer (stream-ordered, like the reference's
    per-stream workspace in src/sglang_exl3/dense.py:45-58) and keeps the old
    one alive for graphs that captured it.

    Growth is refused while the stream is being captured: the zero fill would
    then only run at graph replay, and eager calls on the stream would find
    an uninitialised buffer.  Run each op shape once before capture."""
    key = (device.index or 0, int(torch.cuda.current_stream(device).cuda_stream))
    ws = _WORKSPACES.get(key)
    capturing = torch.cuda.is_current_stream_capturing()
    if ws is None or ws.numel() < nbytes:
        if capturing:
            raise RuntimeError(
                f"sglang_exl3: the workspace of this stream must grow to {nbytes} bytes during HIP graph "
                "capture; run the op once (same shape) on this stream before capturing")
        size = max(nbytes, 1 << 20, 0 if ws is None else 2 * ws.numel())
        if ws is not None and id(ws) in _CAPTURED:
            _RETIRED_WORKSPACES.append((key, ws))
        ws = torch.zeros(size, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    elif capturing:
        _CAPTURED[id(ws)] = ws
    return ws


WAIT_CAUSES = {
    _lib.EXL3_WAIT_MOE_FUSED: "a down item of a one-launch MoE pass (EXL3_MOE_FUSED=1 or EXL3_MOE_FUSED_ROUTED=1) "
                              "stopped waiting for its h blocks",
    _lib.EXL3_WAIT_FAT_TAIL: "the second k-half of a wide-tile GEMM tail tile stopped waiting for the first",
}


def check_waits(device=None) -> None:
    """Raise RuntimeError if a bounded wait inside a launch on one of this
    process's workspaces of `device` (default: the current device) gave up
    since the last check: that launch's output is not valid.  The kernels'
    waits are bounded (about 0.25 s) so that every wave exits; a wait that
    gives up sets a bit of the workspace's status word instead of failing
    silently.  Synchronises the device; not callable during graph capture.
    A workspace whose status was set is zeroed before the error is raised
    (its counters may have been left non-zero), so later calls run clean."""
    import ctypes

    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    torch.cuda.synchronize(idx)
    bits = 0
    bufs = [(k, w) for k, w in _WORKSPACES.items() if k[0] == idx]
    bufs += [(k, w) for k, w in _RETIRED_WORKSPACES if k[0] == idx]
    with torch.cuda.device(idx):
        for _, ws in bufs:
            st = ctypes.c_int32(0)
            rc = _lib.lib().exl3_workspace_status(ws.data_ptr(), ws.numel(), ctypes.byref(st), None)
            _lib.check(rc, "exl3_workspace_status")
            if st.value:
                ws.zero_()
                bits |= st.value
        torch.cuda.synchronize(idx)
    if bits:
        what = "; ".join(v for b, v in WAIT_CAUSES.items() if bits & b) or f"status bits {bits:#x}"
        raise RuntimeError(f"sglang_exl3: a bounded wait gave up ({what}); the outputs of the calls since the "
                           "last check_waits() are not valid")


def check_ws(rc: int, what: str, ws) -> None:
    """Raise for a non-zero status after re-zeroing the workspace the call
    used: a call that failed after some of its launches were enqueued can
    leave split-k counters or fixed-point accumulators non-zero, and every
    later call on the stream relies on them being zero."""
    if rc != _lib.EXL3_OK and ws is not None and not torch.cuda.is_current_stream_capturing():
        ws.zero_()
    _lib.check(rc, what)


def _check_trellis(name: str, trellis: torch.Tensor, K: int) -> None:
    if trellis.dim() != 3 or trellis.dtype != torch.int16:
        raise RuntimeError(f"sglang_exl3::{name}: trellis must be int16 [k/16, n/16, 16*K]")
    if int(trellis.shape[2]) != 16 * int(K):
        raise RuntimeError(
            f"sglang_exl3::{name}: trellis last dim {int(trellis.shape[2])} != 16*K ({16 * int(K)})"
        )


def _f16(name: str, t: torch.Tensor, what: str) -> torch.Tensor:
    if t.dtype != torch.float16:
        raise RuntimeError(f"sglang_exl3::{name}: {what} must be float16 (got {t.dtype})")
    return t.contiguous()


# ------------------------------------------------------------ implementations

def dequant_trellis_impl(trellis, suh, svh, bits, mcg):
    _require_device("dequant_trellis", trellis, suh, svh)
    _check_trellis("dequant_trellis", trellis, bits)
    k, n = int(trellis.shape[0]) * 16, int(trellis.shape[1]) * 16
    suh = _f16("dequant_trellis", suh, "suh")
    svh = _f16("dequant_trellis", svh, "svh")
    if suh.numel() < k or svh.numel() < n:
        raise RuntimeError("sglang_exl3::dequant_trellis: suh/svh are too short")
    tr = trellis.contiguous()
    W = torch.empty((k, n), dtype=torch.float16, device=trellis.device)
    with torch.cuda.device(trellis.device):
        rc = _lib.lib().exl3_dequant_trellis(
            tr.data_ptr(), suh.data_ptr(), svh.data_ptr(), W.data_ptr(), k, n, int(bits),
            _lib.codebook_from_mcg(bool(mcg)), _stream_ptr(trellis))
    _lib.check(rc, "exl3_dequant_trellis")
    return W


def _gemv_like(name, fn, x, trellis, suh, svh, K, cb, max_rows=None, gemv=False):
    """y (fp16 [rows, n]) = x (fp16 [..., k]) @ W through `fn` (exl3_gemv when
    `gemv`, else exl3_gemm), with the workspace that entry point asks for;
    every shape the kernels trust is checked here first."""
    _require_device(name, x, trellis, suh, svh)
    _check_trellis(name, trellis, K)
    if x.dim() < 2:
        raise RuntimeError(f"sglang_exl3::{name}: x must have shape [..., in_features]")
    kdim = int(x.shape[-1])
    m = x.numel() // kdim if kdim else 0
    if kdim != int(trellis.shape[0]) * 16:
        raise RuntimeError(f"sglang_exl3::{name}: x feature dimension does not match trellis")
    if max_rows is not None and not (1 <= m <= max_rows):
        raise RuntimeError(f"sglang_exl3::{name}: native GEMV supports 1 <= m <= {max_rows} (m={m})")
    if cb not in (_lib.CB_3INST, _lib.CB_MCG, _lib.CB_MUL1):
        raise RuntimeError(f"sglang_exl3::{name}: codebook id {cb} outside 0..2")
    x2 = _f16(name, x, "x").reshape(m, kdim)
    n = int(trellis.shape[1]) * 16
    suh = _f16(name, suh, "suh")
    svh = _f16(name, svh, "svh")
    if suh.numel() < kdim or svh.numel() < n:
        raise RuntimeError(f"sglang_exl3::{name}: suh needs {kdim} and svh {n} elements "
                           f"(got {suh.numel()}, {svh.numel()})")
    tr = trellis.contiguous()
    y = torch.empty((m, n), dtype=torch.float16, device=x.device)
    if m == 0:
        return y
    lib = _lib.lib()
    with torch.cuda.device(x.device):
        need = int(lib.exl3_gemv_workspace_size(m, kdim, n, int(K), 1) if gemv
                   else lib.exl3_gemm_workspace_size(m, kdim, n, int(K)))
        ws = workspace(x.device, need) if need else None
        rc = fn(x2.data_ptr(), tr.data_ptr(), suh.data_ptr(), svh.data_ptr(), y.data_ptr(), m, kdim, n,
                int(K), int(cb), 0 if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(),
                _stream_ptr(x))
    check_ws(rc, name, ws)
    return y


def exl3_gemv_impl(x, trellis, suh, svh, K, mcg, mmode=1):
    if mmode not in (0, 1):
        raise RuntimeError("sglang_exl3::exl3_gemv: mmode must be 0 or 1")
    return _gemv_like("exl3_gemv", _lib.lib().exl3_gemv, x, trellis, suh, svh, K,
                      _lib.codebook_from_mcg(bool(mcg)), max_rows=64, gemv=True)


def exl3_gemm_impl(x, trellis, suh, svh, K, mcg):
    return _gemv_like("exl3_gemm", _lib.lib().exl3_gemm, x, trellis, suh, svh, K, _lib.codebook_from_mcg(bool(mcg)))


def exl3_linear_impl(x, trellis, suh, svh, K, codebook):
    """Dense EXL3 linear for any row count and any codebook id (0 = 3INST,
    1 = MCG, 2 = mul1): the single-flag ops above cannot name 3INST, which
    EXL3LinearMethod needs for packs without a codebook marker
    (src/sglang_exl3/dense.py:151-157)."""
    return _gemv_like("exl3_linear", _lib.lib().exl3_gemm, x, trellis, suh, svh, K, int(codebook))


def p2b_gemv_batched_impl(x, trellis_ptrs, suh_ptrs, svh_ptrs, expert_indices, K, mcg, mmode=1):
    name = "p2b_gemv_batched"
    _require_device(name, x, trellis_ptrs, suh_ptrs, svh_ptrs, expert_indices)
    x = _f16(name, x, "x")
    for t, what in ((trellis_ptrs, "trellis_ptrs"), (suh_ptrs, "suh_ptrs"), (svh_ptrs, "svh_ptrs")):
        if t.dtype != torch.int64 or t.dim() != 1:
            raise RuntimeError(f"sglang_exl3::{name}: {what} must be a 1-D int64 pointer table")
    ids = expert_indices.to(torch.int32).contiguous()
    e = ids.numel()
    kdim = int(x.shape[-1])
    per_expert = x.dim() == 3
    m = int(x.shape[1]) if per_expert else int(x.shape[0])
    if per_expert and int(x.shape[0]) != e:
        raise RuntimeError(f"sglang_exl3::{name}: 3-D x must be [num_active, m, k]")
    n = int(mmode) if int(mmode) > 0 else 2048
    out = torch.empty((e, m, n), dtype=torch.float16, device=x.device)
    if e == 0:
        return out
    lib = _lib.lib()
    with torch.cuda.device(x.device):
        need = int(lib.exl3_gemv_workspace_size(m, kdim, n, int(K), e))
        ws = workspace(x.device, need) if need else None
        rc = lib.exl3_p2b_gemv_batched(
            x.data_ptr(), int(per_expert), trellis_ptrs.contiguous().data_ptr(),
            suh_ptrs.contiguous().data_ptr(), svh_ptrs.contiguous().data_ptr(), ids.data_ptr(), e,
            out.data_ptr(), m, kdim, n, int(K), _lib.codebook_from_mcg(bool(mcg)),
            0 if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(), _stream_ptr(x))
    check_ws(rc, name, ws)
    return out


MOE_TABLE_NAMES = ("gate_trellis", "gate_suh", "gate_svh", "up_trellis", "up_suh", "up_svh",
                   "down_trellis", "down_suh", "down_svh")


def _moe_tables(name, tables):
    if len(tables) != 9:
        raise RuntimeError(f"sglang_exl3::{name}: nine pointer tables expected")
    out = []
    e = None
    for t, what in zip(tables, MOE_TABLE_NAMES):
        if t.dtype != torch.int64 or t.dim() != 1 or t.numel() == 0:
            raise RuntimeError(f"sglang_exl3::{name}: {what} pointer table must be a nonempty 1-D int64 tensor")
        if e is None:
            e = t.numel()
        elif t.numel() != e:
            raise RuntimeError(f"sglang_exl3::{name}: pointer tables must be equally sized")
        out.append(t.contiguous())
    return out, int(e)


def _limit_arg(swiglu_limit) -> float:
    lim = float(swiglu_limit)
    if lim != lim or lim < 0:
        raise RuntimeError("sglang_exl3: SwiGLU limit must be nonnegative (0 or inf disables clipping)")
    return lim


def p2b_fused_moe_impl(x, out, gate_trellis_ptrs, gate_suh_ptrs, gate_svh_ptrs, up_trellis_ptrs, up_suh_ptrs,
                       up_svh_ptrs, down_trellis_ptrs, down_suh_ptrs, down_svh_ptrs, expert_indices,
                       routing_weights, K_gate, K_up, K_down, mcg, intermediate_size=2048, swiglu_limit=0.0):
    """One-token fused MoE (csrc/p2b_moe.cu:417-468 semantics; ABI-2 extras
    intermediate_size / swiglu_limit as in csrc/bindings.cpp:192)."""
    name = "p2b_fused_moe"
    tables = (gate_trellis_ptrs, gate_suh_ptrs, gate_svh_ptrs, up_trellis_ptrs, up_suh_ptrs, up_svh_ptrs,
              down_trellis_ptrs, down_suh_ptrs, down_svh_ptrs)
    _require_device(name, x, out, expert_indices, routing_weights, *tables)
    x = _f16(name, x, "x")
    if out.dtype != torch.float16 or not out.is_contiguous() or tuple(out.shape) != tuple(x.shape):
        raise RuntimeError(f"sglang_exl3::{name}: out must be a contiguous fp16 tensor shaped like x")
    if x.dim() != 2 or int(x.shape[0]) != 1:
        raise RuntimeError(f"sglang_exl3::{name}: one input row [1, hidden] expected")
    ids = expert_indices.reshape(-1).to(torch.int32).contiguous()
    rw = routing_weights.reshape(-1)
    if rw.dtype != torch.float16 or rw.numel() != ids.numel() or ids.numel() == 0:
        raise RuntimeError(f"sglang_exl3::{name}: one fp16 routing weight per (nonempty) expert index")
    rw = rw.contiguous()
    tabs, E = _moe_tables(name, tables)
    hidden, inter = int(x.shape[1]), int(intermediate_size)
    lib = _lib.lib()
    with torch.cuda.device(x.device):
        need = int(lib.exl3_moe_workspace_size(1, ids.numel(), E, hidden, inter))
        ws = workspace(x.device, need)
        rc = lib.exl3_p2b_fused_moe(
            x.data_ptr(), out.data_ptr(), *[t.data_ptr() for t in tabs], E, ids.data_ptr(), rw.data_ptr(),
            ids.numel(), hidden, inter, int(K_gate), int(K_up), int(K_down), _lib.codebook_from_mcg(bool(mcg)),
            _limit_arg(swiglu_limit), ws.data_ptr(), ws.numel(), _stream_ptr(x))
    check_ws(rc, name, ws)
    return out


def exl3_moe_layer_impl(x, topk_ids, topk_weights, gate_trellis_ptrs, gate_suh_ptrs, gate_svh_ptrs,
                        up_trellis_ptrs, up_suh_ptrs, up_svh_ptrs, down_trellis_ptrs, down_suh_ptrs, down_svh_ptrs,
                        K_gate, K_up, K_down, mcg, intermediate_size, swiglu_limit=0.0, codebook=-1):
    """Routed-expert MoE layer for a token batch in one call (no host sync).
    topk_ids: [T, topk] local expert ids (outside [0, E) = skipped);
    topk_weights: [T, topk]; swiglu_limit 0 or inf = no clamp; returns fp16 [T, hidden].
    codebook: 0 = 3INST, 1 = MCG, 2 = mul1; -1 = from `mcg` (MCG or mul1)."""
    name = "exl3_moe_layer"
    tables = (gate_trellis_ptrs, gate_suh_ptrs, gate_svh_ptrs, up_trellis_ptrs, up_suh_ptrs, up_svh_ptrs,
              down_trellis_ptrs, down_suh_ptrs, down_svh_ptrs)
    _require_device(name, x, topk_ids, topk_weights, *tables)
    if x.dim() != 2:
        raise RuntimeError(f"sglang_exl3::{name}: x must be [tokens, hidden]")
    T, hidden = int(x.shape[0]), int(x.shape[1])
    ids = topk_ids.reshape(T, -1)
    topk = int(ids.shape[1])
    ids = ids.to(torch.int32).contiguous()
    w = topk_weights.reshape(T, topk).to(torch.float32).contiguous()
    xh = x.to(torch.float16).contiguous()
    tabs, E = _moe_tables(name, tables)
    out = torch.empty((T, hidden), dtype=torch.float16, device=x.device)
    if T == 0 or topk == 0:
        return out.zero_()
    lim = _limit_arg(swiglu_limit)
    lib = _lib.lib()
    with torch.cuda.device(x.device):
        need = int(lib.exl3_moe_workspace_size(T, topk, E, hidden, int(intermediate_size)))
        ws = workspace(x.device, need)
        rc = lib.exl3_moe_layer(
            xh.data_ptr(), ids.data_ptr(), w.data_ptr(), *[t.data_ptr() for t in tabs], E, out.data_ptr(), T, topk,
            hidden, int(intermediate_size), int(K_gate), int(K_up), int(K_down),
            _lib.codebook_from_mcg(bool(mcg)) if int(codebook) < 0 else int(codebook), lim, ws.data_ptr(),
            ws.numel(), _stream_ptr(x))
    check_ws(rc, name, ws)
    return out


def exl3_gate_up_swiglu_impl(x, suh, gate_trellis, gate_svh, up_trellis, up_svh, K, codebook, swiglu_limit=0.0):
    """fp16 [rows, n] = silu(min(x @ W_gate, L)) * clamp(x @ W_up, -L, L) for x [..., k], both
    projections sharing the input rotation suh (the reference's fused gate/up path rotates once
    with the gate's suh: src/sglang_exl3/exl3.py:1184-1206)."""
    name = "exl3_gate_up_swiglu"
    _require_device(name, x, suh, gate_trellis, gate_svh, up_trellis, up_svh)
    _check_trellis(name, gate_trellis, K)
    _check_trellis(name, up_trellis, K)
    if tuple(gate_trellis.shape) != tuple(up_trellis.shape):
        raise RuntimeError(f"sglang_exl3::{name}: gate and up trellis shapes differ")
    kdim = int(x.shape[-1])
    m = x.numel() // kdim if kdim else 0
    if kdim != int(gate_trellis.shape[0]) * 16:
        raise RuntimeError(f"sglang_exl3::{name}: x feature dimension does not match trellis")
    if int(codebook) not in (_lib.CB_3INST, _lib.CB_MCG, _lib.CB_MUL1):
        raise RuntimeError(f"sglang_exl3::{name}: codebook id {codebook} outside 0..2")
    n = int(gate_trellis.shape[1]) * 16
    x2 = _f16(name, x, "x").reshape(m, kdim)
    suh, gsv, usv = (_f16(name, t, w) for t, w in ((suh, "suh"), (gate_svh, "gate_svh"), (up_svh, "up_svh")))
    if suh.numel() < kdim or gsv.numel() < n or usv.numel() < n:
        raise RuntimeError(f"sglang_exl3::{name}: suh needs {kdim}, svh {n} elements")
    gt, ut = gate_trellis.contiguous(), up_trellis.contiguous()
    out = torch.empty((m, n), dtype=torch.float16, device=x.device)
    if m == 0:
        return out
    lib = _lib.lib()
    with torch.cuda.device(x.device):
        need = int(lib.exl3_gate_up_workspace_size(m, kdim, n, int(K)))
        ws = workspace(x.device, need)
        rc = lib.exl3_gate_up_swiglu(x2.data_ptr(), suh.data_ptr(), gt.data_ptr(), gsv.data_ptr(), ut.data_ptr(),
                                     usv.data_ptr(), out.data_ptr(), m, kdim, n, int(K), int(codebook),
                                     _limit_arg(swiglu_limit), ws.data_ptr(), ws.numel(), _stream_ptr(x))
    check_ws(rc, name, ws)
    return out


def _fat_common(name, a, packed, out, svh, K):
    _require_device(name, a, packed, out, svh)
    if a.dtype != torch.float16 or a.dim() != 2 or not a.is_contiguous():
        raise RuntimeError(f"sglang_exl3::{name}: a must be a contiguous fp16 [M, k] tensor")
    _check_trellis(name, packed, K)
    if not packed.is_contiguous() or not svh.is_contiguous() or not out.is_contiguous():
        raise RuntimeError(f"sglang_exl3::{name}: tensors must be contiguous")
    if out.dtype != torch.float32 or out.dim() != 2:
        raise RuntimeError(f"sglang_exl3::{name}: out must be float32 [rows, N]")
    if svh.dtype != torch.float16 or svh.dim() != 1:
        raise RuntimeError(f"sglang_exl3::{name}: svh must be a float16 vector")
    M, k = int(a.shape[0]), int(a.shape[1])
    n = int(svh.numel())
    if k != int(packed.shape[0]) * 16 or n != int(packed.shape[1]) * 16:
        raise RuntimeError(f"sglang_exl3::{name}: a / svh do not match the packed tensor")
    if int(out.shape[1]) != n:
        raise RuntimeError(f"sglang_exl3::{name}: out N dimension mismatch")
    return M, k, n


def exl3_fat_gemm_impl(a, packed, out, svh, K, mcg, mul1):
    """out (fp32 [M, N]) = svh * H(a . T) / sqrt(128), a rotated (csrc/exl3_fat_gemm.cu:275-287)."""
    name = "exl3_fat_gemm"
    M, k, n = _fat_common(name, a, packed, out, svh, K)
    if tuple(out.shape) != (M, n):
        raise RuntimeError(f"sglang_exl3::{name}: out shape must be [M, N]")
    with torch.cuda.device(a.device):
        rc = _lib.lib().exl3_fat_gemm(a.data_ptr(), packed.data_ptr(), out.data_ptr(), svh.data_ptr(), M, k, n,
                                      int(K), _lib.codebook_id(bool(mcg), bool(mul1)), _stream_ptr(a))
    _lib.check(rc, name)


def exl3_fat_gemm_scatter_impl(a, packed, out, svh, token_idx, route_weight, K, mcg, mul1):
    """out[token_idx[m]] += route_weight[m] * (svh * H(a . T)[m] / sqrt(128)) (csrc/exl3_fat_gemm.cu:289-305)."""
    name = "exl3_fat_gemm_scatter"
    M, k, n = _fat_common(name, a, packed, out, svh, K)
    _require_device(name, a, token_idx, route_weight)
    if token_idx.dtype != torch.int64 or route_weight.dtype != torch.float16:
        raise RuntimeError(f"sglang_exl3::{name}: token_idx must be int64 and route_weight float16")
    if token_idx.numel() != M or route_weight.numel() != M:
        raise RuntimeError(f"sglang_exl3::{name}: routing tensors must have M elements")
    ti, rw = token_idx.contiguous(), route_weight.contiguous()
    with torch.cuda.device(a.device):
        rc = _lib.lib().exl3_fat_gemm_scatter(a.data_ptr(), packed.data_ptr(), out.data_ptr(), svh.data_ptr(),
                                              ti.data_ptr(), rw.data_ptr(), M, k, n, int(K),
                                              _lib.codebook_id(bool(mcg), bool(mul1)), _stream_ptr(a))
    _lib.check(rc, name)


# ----------------------------------------------------------------- registry

def register_custom_ops() -> bool:
    """Register the EXL3 kernels in torch.ops.sglang_exl3 with fake kernels
    (same schemas as src/sglang_exl3/ops.py:38-226)."""
    global _OPS_REGISTERED
    if _OPS_REGISTERED:
        return True

    @torch.library.custom_op("sglang_exl3::dequant_trellis", mutates_args=())
    def dequant_trellis(trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor, bits: int,
                        mcg: bool) -> torch.Tensor:
        return dequant_trellis_impl(trellis, suh, svh, bits, mcg)

    @dequant_trellis.register_fake
    def _(trellis, suh, svh, bits, mcg):
        return torch.empty((trellis.size(0) * 16, trellis.size(1) * 16), dtype=torch.float16,
                           device=trellis.device)

    @torch.library.custom_op("sglang_exl3::exl3_gemv", mutates_args=())
    def exl3_gemv(x: torch.Tensor, trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor, K: int,
                  mcg: bool, mmode: int = 1) -> torch.Tensor:
        return exl3_gemv_impl(x, trellis, suh, svh, K, mcg, mmode)

    @exl3_gemv.register_fake
    def _(x, trellis, suh, svh, K, mcg, mmode=1):
        out_dim = svh.size(0) if svh.ndim == 1 else trellis.size(1) * 16
        return torch.empty((x.shape[0], out_dim), dtype=x.dtype, device=x.device)

    @torch.library.custom_op("sglang_exl3::exl3_gemm", mutates_args=())
    def exl3_gemm(x: torch.Tensor, trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor, K: int,
                  mcg: bool) -> torch.Tensor:
        return exl3_gemm_impl(x, trellis, suh, svh, K, mcg)

    @exl3_gemm.register_fake
    def _(x, trellis, suh, svh, K, mcg):
        out_dim = svh.size(0) if svh.ndim == 1 else trellis.size(1) * 16
        return torch.empty((x.shape[0], out_dim), dtype=x.dtype, device=x.device)

    @torch.library.custom_op("sglang_exl3::exl3_linear", mutates_args=())
    def exl3_linear(x: torch.Tensor, trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor, K: int,
                    codebook: int) -> torch.Tensor:
        return exl3_linear_impl(x, trellis, suh, svh, K, codebook)

    @exl3_linear.register_fake
    def _(x, trellis, suh, svh, K, codebook):
        rows = x.numel() // x.shape[-1] if x.shape[-1] else 0
        return torch.empty((rows, trellis.size(1) * 16), dtype=torch.float16, device=x.device)

    @torch.library.custom_op("sglang_exl3::p2b_gemv_batched", mutates_args=())
    def p2b_gemv_batched(x: torch.Tensor, trellis_ptrs: torch.Tensor, suh_ptrs: torch.Tensor,
                         svh_ptrs: torch.Tensor, expert_indices: torch.Tensor, K: int, mcg: bool,
                         mmode: int = 1) -> torch.Tensor:
        return p2b_gemv_batched_impl(x, trellis_ptrs, suh_ptrs, svh_ptrs, expert_indices, K, mcg, mmode)

    @p2b_gemv_batched.register_fake
    def _(x, trellis_ptrs, suh_ptrs, svh_ptrs, expert_indices, K, mcg, mmode=1):
        e = expert_indices.numel()
        m = x.size(1) if x.dim() == 3 else x.size(0)
        n = mmode if mmode > 0 else 2048
        return torch.empty((e, m, n), dtype=x.dtype, device=x.device)

    @torch.library.custom_op("sglang_exl3::p2b_fused_moe", mutates_args=("out",))
    def p2b_fused_moe(x: torch.Tensor, out: torch.Tensor, gate_trellis_ptrs: torch.Tensor,
                      gate_suh_ptrs: torch.Tensor, gate_svh_ptrs: torch.Tensor, up_trellis_ptrs: torch.Tensor,
                      up_suh_ptrs: torch.Tensor, up_svh_ptrs: torch.Tensor, down_trellis_ptrs: torch.Tensor,
                      down_suh_ptrs: torch.Tensor, down_svh_ptrs: torch.Tensor, expert_indices: torch.Tensor,
                      routing_weights: torch.Tensor, K_gate: int, K_up: int, K_down: int,
                      mcg: bool) -> None:
        p2b_fused_moe_impl(x, out, gate_trellis_ptrs, gate_suh_ptrs, gate_svh_ptrs, up_trellis_ptrs,
                           up_suh_ptrs, up_svh_ptrs, down_trellis_ptrs, down_suh_ptrs, down_svh_ptrs,
                           expert_indices, routing_weights, K_gate, K_up, K_down, mcg)

    @p2b_fused_moe.register_fake
    def _(x, out, gate_trellis_ptrs, gate_suh_ptrs, gate_svh_ptrs, up_trellis_ptrs, up_suh_ptrs, up_svh_ptrs,
          down_trellis_ptrs, down_suh_ptrs, down_svh_ptrs, expert_indices, routing_weights, K_gate, K_up,
          K_down, mcg):
        return None

    @torch.library.custom_op("sglang_exl3::exl3_moe_layer", mutates_args=())
    def exl3_moe_layer(x: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor,
                       gate_trellis_ptrs: torch.Tensor, gate_suh_ptrs: torch.Tensor, gate_svh_ptrs: torch.Tensor,
                       up_trellis_ptrs: torch.Tensor, up_suh_ptrs: torch.Tensor, up_svh_ptrs: torch.Tensor,
                       down_trellis_ptrs: torch.Tensor, down_suh_ptrs: torch.Tensor, down_svh_ptrs: torch.Tensor,
                       K_gate: int, K_up: int, K_down: int, mcg: bool, intermediate_size: int,
                       swiglu_limit: float = 0.0, codebook: int = -1) -> torch.Tensor:
        return exl3_moe_layer_impl(x, topk_ids, topk_weights, gate_trellis_ptrs, gate_suh_ptrs, gate_svh_ptrs,
                                   up_trellis_ptrs, up_suh_ptrs, up_svh_ptrs, down_trellis_ptrs, down_suh_ptrs,
                                   down_svh_ptrs, K_gate, K_up, K_down, mcg, intermediate_size, swiglu_limit,
                                   codebook)

    @exl3_moe_layer.register_fake
    def _(x, topk_ids, topk_weights, *rest):
        return torch.empty((x.shape[0], x.shape[1]), dtype=torch.float16, device=x.device)

    @torch.library.custom_op("sglang_exl3::exl3_gate_up_swiglu", mutates_args=())
    def exl3_gate_up_swiglu(x: torch.Tensor, suh: torch.Tensor, gate_trellis: torch.Tensor, gate_svh: torch.Tensor,
                            up_trellis: torch.Tensor, up_svh: torch.Tensor, K: int, codebook: int,
                            swiglu_limit: float = 0.0) -> torch.Tensor:
        return exl3_gate_up_swiglu_impl(x, suh, gate_trellis, gate_svh, up_trellis, up_svh, K, codebook,
                                        swiglu_limit)

    @exl3_gate_up_swiglu.register_fake
    def _(x, suh, gate_trellis, gate_svh, up_trellis, up_svh, K, codebook, swiglu_limit=0.0):
        rows = x.numel() // x.shape[-1] if x.shape[-1] else 0
        return torch.empty((rows, gate_trellis.size(1) * 16), dtype=torch.float16, device=x.device)

    @torch.library.custom_op("sglang_exl3::exl3_fat_gemm", mutates_args=("out",))
    def exl3_fat_gemm(a: torch.Tensor, packed: torch.Tensor, out: torch.Tensor, svh: torch.Tensor, K: int,
                      mcg: bool, mul1: bool) -> None:
        exl3_fat_gemm_impl(a, packed, out, svh, K, mcg, mul1)

    @exl3_fat_gemm.register_fake
    def _(a, packed, out, svh, K, mcg, mul1):
        return None

    @torch.library.custom_op("sglang_exl3::exl3_fat_gemm_scatter", mutates_args=("out",))
    def exl3_fat_gemm_scatter(a: torch.Tensor, packed: torch.Tensor, out: torch.Tensor, svh: torch.Tensor,
                              token_idx: torch.Tensor, route_weight: torch.Tensor, K: int, mcg: bool,
                              mul1: bool) -> None:
        exl3_fat_gemm_scatter_impl(a, packed, out, svh, token_idx, route_weight, K, mcg, mul1)

    @exl3_fat_gemm_scatter.register_fake
    def _(a, packed, out, svh, token_idx, route_weight, K, mcg, mul1):
        return None

    _OPS_REGISTERED = True
    logger.info("registered sglang_exl3 custom ops (gfx950 HIP backend)")
    return True
