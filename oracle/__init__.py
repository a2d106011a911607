"""CPU oracle for the EXL3 quantized-matmul path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker (never as the thing
measured or shipped).  The product package ``sglang_exl3`` never imports it.

Two libraries sit behind it:

* ``_build/libexl3_oracle.so`` — ``exl3_oracle.c``, a C restatement of the
  reference's host decode (``csrc/exl3_dequant.cuh:10-148``), dequant
  (``csrc/bindings.cpp:15-100``) and CPU GEMV path (``csrc/bindings.cpp:144-146``).
* ``_ref/libexl3_ref.so`` — the reference's own header compiled where it lies
  (``oracle/ref_shim.cpp``); used to pin the restatement.  Absent on machines
  without ``/root/reference`` unless built beforehand.

Every function the oracle exposes is pinned by a test in
``tests/test_oracle.py``: against the compiled reference header (codebook
tables, windows, FWHT), the committed golden vectors, closed forms (all-zero
trellis, single-window tiles, Sylvester-matrix identity) and brute force.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_ORACLE_SO = os.path.join(_HERE, "_build", "libexl3_oracle.so")
_REF_SO = os.path.join(_HERE, "_ref", "libexl3_ref.so")

_P = ctypes.c_void_p
_lib = None
_ref = None


def build(force: bool = False) -> None:
    """Compile the C oracle (and the reference-header shim when the reference
    tree is present) with gcc via oracle/Makefile."""
    if force or not os.path.exists(_ORACLE_SO) or os.path.exists("/root/reference"):
        subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_ORACLE_SO):
            build()
        L = ctypes.CDLL(_ORACLE_SO)
        L.orc_half_to_float.restype = ctypes.c_float
        L.orc_half_to_float.argtypes = [ctypes.c_uint16]
        L.orc_float_to_half_rtz.restype = ctypes.c_uint16
        L.orc_float_to_half_rtz.argtypes = [ctypes.c_float]
        L.orc_float_to_half_rne.restype = ctypes.c_uint16
        L.orc_float_to_half_rne.argtypes = [ctypes.c_float]
        L.orc_read_window.restype = ctypes.c_uint16
        L.orc_read_window.argtypes = [_P, ctypes.c_size_t, ctypes.c_size_t]
        L.orc_codebook_exact.restype = ctypes.c_float
        L.orc_codebook_exact.argtypes = [ctypes.c_uint16, ctypes.c_int]
        L.orc_decode_state.restype = ctypes.c_uint16
        L.orc_decode_state.argtypes = [ctypes.c_uint16, ctypes.c_int, ctypes.c_int]
        L.orc_codebook_table.argtypes = [ctypes.c_int, ctypes.c_int, _P]
        L.orc_decode_tile.argtypes = [_P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P]
        L.orc_fwht.argtypes = [_P, ctypes.c_int]
        L.orc_dequant.restype = ctypes.c_int
        L.orc_dequant.argtypes = [_P, _P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                  ctypes.c_int, ctypes.c_int, _P]
        L.orc_matmul_f16.argtypes = [_P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P]
        L.orc_cpu_gemv.restype = ctypes.c_int
        L.orc_cpu_gemv.argtypes = [_P, _P, _P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                   ctypes.c_int, ctypes.c_int, _P, _P]
        L.orc_had_rows.argtypes = [_P, ctypes.c_int, ctypes.c_int, _P, _P, ctypes.c_float, _P]
        L.orc_swiglu.restype = ctypes.c_float
        L.orc_swiglu.argtypes = [ctypes.c_float, ctypes.c_float, ctypes.c_float]
        _lib = L
    return _lib


def ref_lib():
    """The reference's compiled host header, or None when it was never built."""
    global _ref
    if _ref is None:
        if not os.path.exists(_REF_SO):
            try:
                build()
            except Exception:
                return None
        if not os.path.exists(_REF_SO):
            return None
        R = ctypes.CDLL(_REF_SO)
        R.ref_read_window.restype = ctypes.c_uint16
        R.ref_read_window.argtypes = [_P, ctypes.c_size_t, ctypes.c_size_t]
        R.ref_decode_codebook_bits.restype = ctypes.c_uint16
        R.ref_decode_codebook_bits.argtypes = [ctypes.c_uint16, ctypes.c_int]
        R.ref_float_to_half_bits.restype = ctypes.c_uint16
        R.ref_float_to_half_bits.argtypes = [ctypes.c_float]
        R.ref_half_bits_to_float.restype = ctypes.c_float
        R.ref_half_bits_to_float.argtypes = [ctypes.c_uint16]
        R.ref_lop3_6a.restype = ctypes.c_uint32
        R.ref_lop3_6a.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]
        R.ref_hadamard.argtypes = [_P, ctypes.c_int]
        R.ref_decode_weight.restype = ctypes.c_float
        R.ref_decode_weight.argtypes = [_P, ctypes.c_size_t, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        _ref = R
    return _ref


# ---------------------------------------------------------------- wrappers

def codebook_table(cb: int, rtz: bool) -> np.ndarray:
    out = np.empty(65536, dtype=np.uint16)
    lib().orc_codebook_table(cb, int(rtz), _ptr(out))
    return out


def read_window(tile16: np.ndarray, bit: int) -> int:
    t = np.ascontiguousarray(tile16, dtype=np.uint16)
    return int(lib().orc_read_window(_ptr(t), t.size, bit))


def decode_tile(tile16: np.ndarray, K: int, cb: int, rtz: bool) -> np.ndarray:
    t = np.ascontiguousarray(tile16, dtype=np.uint16)
    assert t.size == 16 * K
    out = np.empty((16, 16), dtype=np.uint16)
    lib().orc_decode_tile(_ptr(t), K, cb, int(rtz), _ptr(out))
    return out


def fwht(v: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(v, dtype=np.float32).copy()
    lib().orc_fwht(_ptr(a), a.size)
    return a


def dequant(trellis: np.ndarray, suh: np.ndarray, svh: np.ndarray, K: int, cb: int,
            rtz: bool = True) -> np.ndarray:
    """W[k, n] as fp16 bit patterns (uint16).  trellis: int16/uint16 [k/16, n/16, 16K];
    suh/svh: fp16 (or their uint16 bits)."""
    tr = np.ascontiguousarray(trellis).view(np.uint16)
    su = np.ascontiguousarray(suh).view(np.uint16)
    sv = np.ascontiguousarray(svh).view(np.uint16)
    k, n = tr.shape[0] * 16, tr.shape[1] * 16
    assert tr.shape[2] == 16 * K
    W = np.empty((k, n), dtype=np.uint16)
    rc = lib().orc_dequant(_ptr(tr), _ptr(su), _ptr(sv), k, n, K, cb, int(rtz), _ptr(W))
    if rc:
        raise ValueError(f"orc_dequant failed rc={rc}")
    return W


def matmul(x16: np.ndarray, W16: np.ndarray) -> np.ndarray:
    """fp32 result of x[m,k] @ W[k,n] for fp16 operands (fp64 accumulation)."""
    x = np.ascontiguousarray(x16).view(np.uint16)
    W = np.ascontiguousarray(W16).view(np.uint16)
    m, k = x.shape
    n = W.shape[1]
    y = np.empty((m, n), dtype=np.float32)
    lib().orc_matmul_f16(_ptr(x), _ptr(W), m, k, n, _ptr(y))
    return y


def cpu_gemv(x16: np.ndarray, trellis: np.ndarray, suh: np.ndarray, svh: np.ndarray, K: int,
             cb: int, W_scratch: Optional[np.ndarray] = None) -> np.ndarray:
    """The reference's CPU exl3_gemv: truncating dequant + fp32 GEMM (one thread)."""
    x = np.ascontiguousarray(x16).view(np.uint16)
    tr = np.ascontiguousarray(trellis).view(np.uint16)
    su = np.ascontiguousarray(suh).view(np.uint16)
    sv = np.ascontiguousarray(svh).view(np.uint16)
    m, k = x.shape
    n = tr.shape[1] * 16
    if W_scratch is None:
        W_scratch = np.empty((k, n), dtype=np.uint16)
    y = np.empty((m, n), dtype=np.float32)
    rc = lib().orc_cpu_gemv(_ptr(x), _ptr(tr), _ptr(su), _ptr(sv), m, k, n, K, cb,
                            _ptr(W_scratch), _ptr(y))
    if rc:
        raise ValueError(f"orc_cpu_gemv failed rc={rc}")
    return y


def had_rows(x: np.ndarray, pre: Optional[np.ndarray], post: Optional[np.ndarray],
             r: float = 0.088388347648) -> np.ndarray:
    a = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = a.shape
    y = np.empty_like(a)
    pre_b = None if pre is None else np.ascontiguousarray(pre).view(np.uint16)
    post_b = None if post is None else np.ascontiguousarray(post).view(np.uint16)
    lib().orc_had_rows(_ptr(a), rows, cols, None if pre_b is None else _ptr(pre_b),
                       None if post_b is None else _ptr(post_b), r, _ptr(y))
    return y


def round_bf16(a: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 (ties to even), returned as float32 (finite inputs)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def round_to(a: np.ndarray, dtype: str) -> np.ndarray:
    """float32 values rounded to dtype ("f16", "bf16", "f32"), returned as float32."""
    a = np.asarray(a, dtype=np.float32)
    if dtype == "f16":
        return a.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        return round_bf16(a)
    return a


def sylvester(n: int = 128) -> np.ndarray:
    """Unnormalised Sylvester-Hadamard matrix built by the reference's doubling
    [[H, H], [H, -H]] (src/sglang_exl3/hadamard_cache.py:105-108)."""
    H = np.ones((1, 1))
    while H.shape[0] < n:
        H = np.block([[H, H], [H, -H]])
    return H


def had_fast(x: np.ndarray, post: Optional[np.ndarray], dtype: str) -> np.ndarray:
    """transform_hadamard_fast (src/sglang_exl3/hadamard_cache.py:88-120) in
    dtype ("f16", "bf16", "f32"): each 128-block times the Sylvester matrix of
    +-h, h = 1/sqrt(128) rounded to fp32 and then to dtype (:109), the block
    sum taken exactly (float64: the products x h are exact, and so is the sum
    of 128 of them for operands of a few binades) and rounded to fp32, then to
    dtype (the matmul's output); then times post (suh converted to dtype, :116)
    and rounded to dtype again.  x holds dtype values as float32."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = a.shape
    h = float(round_to(np.float32([1.0 / 128.0 ** 0.5]), dtype)[0])
    blocks = a.astype(np.float64).reshape(rows, cols // 128, 128)
    s = np.einsum("rbi,ij->rbj", blocks, sylvester() * h).reshape(rows, cols)
    y = round_to(s.astype(np.float32), dtype)
    if post is not None:
        y = round_to(y * round_to(np.asarray(post, dtype=np.float32), dtype), dtype)
    return y


def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(bits).view(np.float16).astype(np.float32)


# ---------------------------------------------------------- layer-level refs

def linear_ref(x: np.ndarray, trellis: np.ndarray, suh: np.ndarray, svh: np.ndarray, K: int,
               cb: int) -> np.ndarray:
    """fp32 reference of an EXL3 linear: x (fp16) @ dequant(W) with fp64 accumulation."""
    W = dequant(trellis, suh, svh, K, cb, rtz=True)
    x16 = np.ascontiguousarray(x, dtype=np.float16)
    return matmul(x16, W)


def swiglu(g: np.ndarray, u: np.ndarray, limit: float) -> np.ndarray:
    g = g.astype(np.float32)
    u = u.astype(np.float32)
    if limit > 0 and np.isfinite(limit):
        g = np.minimum(g, np.float32(limit))
        u = np.clip(u, -np.float32(limit), np.float32(limit))
    return (g / (np.float32(1.0) + np.exp(-g)) * u).astype(np.float32)


def moe_ref(x: np.ndarray, topk_ids: np.ndarray, topk_w: np.ndarray, experts: list,
            limit: float = float("inf")) -> np.ndarray:
    """Routed-expert MoE in fp32 following the reference's python loop
    (src/sglang_exl3/exl3.py:520-576): per expert, gate/up linears on the fp16
    tokens, SwiGLU, the activation cast to fp16 for the down linear, then
    out[t] += w * down.  `experts[e]` = dict(gate=(trellis,suh,svh,K,cb), up=..., down=...).
    Ids outside [0, len(experts)) are skipped."""
    T, H = x.shape
    out = np.zeros((T, H), dtype=np.float32)
    ids = np.asarray(topk_ids)
    w = np.asarray(topk_w, dtype=np.float32)
    x16 = np.ascontiguousarray(x, dtype=np.float16)
    used = [e for e in sorted(set(int(i) for i in ids.reshape(-1))) if 0 <= e < len(experts)]
    # the dequants are independent C calls (ctypes releases the GIL): run them
    # on a few threads, then the loop below in expert order as before
    jobs = [(e, p) for e in used for p in ("gate", "up", "down")]

    def _dq(job):
        e, p = job
        spec = experts[e][p]
        return dequant(*spec[:3], spec[3], spec[4], rtz=True)

    from concurrent.futures import ThreadPoolExecutor

    with ThreadPoolExecutor(max_workers=max(1, min(16, os.cpu_count() or 1))) as ex:
        mats = list(ex.map(_dq, jobs))
    cache = {}
    for (e, p), W in zip(jobs, mats):
        cache.setdefault(e, {})[p] = W
    for e in used:
        tok, slot = np.nonzero(ids == e)
        h = x16[tok]
        Wg, Wu, Wd = cache[e]["gate"], cache[e]["up"], cache[e]["down"]
        g = matmul(h, Wg)
        u = matmul(h, Wu)
        act = swiglu(g, u, limit).astype(np.float16)
        d = matmul(act, Wd)
        np.add.at(out, tok, d * w[tok, slot][:, None])
    return out
