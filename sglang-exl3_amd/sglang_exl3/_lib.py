"""ctypes binding of the gfx950 HIP library (libsglang_exl3_amd.so).

The C ABI is declared in include/sglang_exl3_amd.h.  There is no fallback:
if the library is missing or fails to load, every op raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("SGLANG_EXL3_AMD_LIB", os.path.join(_HERE, "_lib", "libsglang_exl3_amd.so"))

EXL3_OK = 0
EXL3_ERR_ARG = 1
EXL3_ERR_UNSUPPORTED = 2
EXL3_ERR_HIP = 3
EXL3_ERR_WORKSPACE = 4

# bits of the workspace status word (exl3_workspace_status)
EXL3_WAIT_MOE_FUSED = 1
EXL3_WAIT_FAT_TAIL = 2

# element types of exl3_hadamard_fast
DTYPE_F16 = 0
DTYPE_BF16 = 1
DTYPE_F32 = 2

CB_3INST = 0
CB_MCG = 1
CB_MUL1 = 2

_P = ctypes.c_void_p
_I = ctypes.c_int
_SZ = ctypes.c_size_t
_F = ctypes.c_float

# name -> (restype, argtypes); exactly the entry points include/sglang_exl3_amd.h declares
SIGNATURES = {
    "exl3_abi_version": (_I, []),
    "exl3_last_error": (ctypes.c_char_p, []),
    "exl3_dequant_trellis": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "exl3_decode_states": (_I, [_P, _I, _I, _I, _P, _P]),
    "exl3_decode_tiles": (_I, [_P, _P, _I, _I, _I, _I, _I, _P]),
    "exl3_gemv_workspace_size": (_SZ, [_I, _I, _I, _I, _I]),
    "exl3_gemv_plan": (_I, [_I, _I, _I, _I, _I, _P]),
    "exl3_gemv": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _SZ, _P]),
    "exl3_gemv_noalloc": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "exl3_gemm": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _SZ, _P]),
    "exl3_p2b_gemv_batched": (_I, [_P, _I, _P, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I, _P, _SZ, _P]),
    "exl3_hadamard_rows": (_I, [_P, _P, _P, _P, _F, _I, _I, _P]),
    "exl3_hadamard_fast": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "exl3_gemm_workspace_size": (_SZ, [_I, _I, _I, _I]),
    "exl3_fat_gemm": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "exl3_fat_gemm_scatter": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "exl3_gate_up_workspace_size": (_SZ, [_I, _I, _I, _I]),
    "exl3_gate_up_swiglu": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _P, _SZ, _P]),
    "exl3_moe_workspace_size": (_SZ, [_I, _I, _I, _I, _I]),
    "exl3_moe_plan": (_I, [_I, _I, _I, _I, _I, _P]),
    "exl3_moe_layer": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _P, _I, _I, _I, _I,
                            _I, _I, _I, _I, _F, _P, _SZ, _P]),
    "exl3_p2b_fused_moe": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I,
                                _I, _I, _I, _I, _F, _P, _SZ, _P]),
    "exl3_workspace_status": (_I, [_P, _SZ, _P, _P]),
}

_lib = None
_lock = threading.Lock()


class Exl3Error(RuntimeError):
    """A non-zero status from the HIP library."""


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"sglang_exl3 HIP library not found at {LIB_PATH}; build it with "
                    "`python sglang-exl3_amd/build_hip.py` (or __graft_entry__.build())"
                )
            L = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(L, name)
                fn.restype = res
                fn.argtypes = args
            _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    if rc != EXL3_OK:
        msg = lib().exl3_last_error()
        raise Exl3Error(f"{what} failed (status {rc}): {msg.decode() if msg else ''}")


def codebook_id(mcg: bool, mul1: bool = False) -> int:
    """Codebook of the two-flag ops (exl3_fat_gemm): mcg -> 1, mul1 -> 2,
    neither -> 0 (3INST), as exllamav3 selects it."""
    if mcg and mul1:
        raise ValueError("EXL3 tensor cannot use both mcg and mul1")
    return CB_MCG if mcg else (CB_MUL1 if mul1 else CB_3INST)


def codebook_from_mcg(mcg: bool) -> int:
    """Codebook of the single-flag ops (dequant_trellis, exl3_gemv, exl3_gemm,
    p2b_*): the reference passes `mcg ? 1 : 2` (csrc/bindings.cpp:48,
    csrc/exl3_gemv.cu:32), so False selects mul1."""
    return CB_MCG if mcg else CB_MUL1
