"""Shared helpers of the GPU parity tests: seeded EXL3 weights and the tolerance bar."""

from __future__ import annotations

import numpy as np
import torch

# Tolerance bar of the matmul outputs: max-abs-err <= 2e-2 * rms(ref)
# and cosine >= 0.9999 against an fp32-accumulated reference on the same inputs.
MAX_ABS_REL_RMS = 2e-2
MIN_COSINE = 0.9999

CB_IDS = {"3inst": 0, "mcg": 1, "mul1": 2}


def make_weight(k: int, n: int, K: int, seed: int):
    """Seeded EXL3 weight: uniform random int16 trellis (every 16-bit state reachable)
    and +-1 fp16 sign vectors.  numpy arrays."""
    rng = np.random.default_rng(seed)
    trellis = rng.integers(-32768, 32768, size=(k // 16, n // 16, 16 * K), dtype=np.int64).astype(np.int16)
    suh = np.where(rng.random(k) < 0.5, -1.0, 1.0).astype(np.float16)
    svh = np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float16)
    return trellis, suh, svh


def make_x(m: int, k: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed + 7919)
    return rng.standard_normal((m, k)).astype(np.float16)


def to_dev(*arrs, device="cuda"):
    return [torch.from_numpy(np.ascontiguousarray(a)).to(device) for a in arrs]


def check_close(out: np.ndarray, ref: np.ndarray, what: str = "") -> dict:
    out = np.asarray(out, dtype=np.float64).reshape(-1)
    ref = np.asarray(ref, dtype=np.float64).reshape(-1)
    assert np.all(np.isfinite(out)), f"{what}: non-finite output"
    rms = float(np.sqrt(np.mean(ref * ref)))
    err = float(np.max(np.abs(out - ref)))
    cos = float(np.dot(out, ref) / (np.linalg.norm(out) * np.linalg.norm(ref) + 1e-300))
    assert err <= MAX_ABS_REL_RMS * rms, f"{what}: max-abs-err {err:.4g} > {MAX_ABS_REL_RMS} * rms {rms:.4g}"
    assert cos >= MIN_COSINE, f"{what}: cosine {cos:.6f} < {MIN_COSINE}"
    return {"max_abs_err": err, "rms": rms, "cos": cos}
