"""Write the golden vectors of the EXL3 decode path from the reference's own code.

Run in a container where /root/reference exists (it builds oracle/_ref from the
reference header csrc/exl3_dequant.cuh in place).  Everything written here is
data: inputs and the outputs the reference's functions give for them.

  codebooks.npz   sha256 of the 65536-entry truncating codebook tables
                  (decode_codebook_bits, csrc/exl3_dequant.cuh:74-93) for
                  cb 0/1/2, plus 4096 sampled (state, bits) pairs per codebook
  windows.npz     random tiles for K = 1..8 with read_window at every stream bit
                  (csrc/exl3_dequant.cuh:110-128)
  dequant.npz     small seeded weights and their dequantised W bits, composed
                  from the reference's decode_weight / hadamard /
                  float_to_half_bits in the order of dequant_cpu
                  (csrc/bindings.cpp:15-100: lane/peer swizzle, row FWHT * norm,
                  column FWHT, ((v * norm) * suh) * svh, RNE fp16)

Usage: python tests/golden/make_golden.py
"""

from __future__ import annotations

import ctypes
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402

NORM = np.float32(0.08838834764831845)


def ref():
    R = oracle.ref_lib()
    if R is None:
        raise SystemExit("reference header build (oracle/_ref) unavailable: run where /root/reference exists")
    return R


def codebooks(R):
    out = {}
    rng = np.random.default_rng(11)
    for cb in (0, 1, 2):
        table = np.array([R.ref_decode_codebook_bits(s, cb) for s in range(65536)], dtype=np.uint16)
        out[f"sha256_cb{cb}"] = np.frombuffer(hashlib.sha256(table.tobytes()).digest(), dtype=np.uint8)
        idx = np.sort(rng.choice(65536, size=4096, replace=False)).astype(np.uint16)
        out[f"states_cb{cb}"] = idx
        out[f"bits_cb{cb}"] = table[idx]
    np.savez_compressed(os.path.join(HERE, "codebooks.npz"), **out)


def windows(R):
    out = {}
    rng = np.random.default_rng(12)
    for K in range(1, 9):
        tile = rng.integers(0, 65536, size=16 * K, dtype=np.uint16)
        w = np.array([R.ref_read_window(tile.ctypes.data, tile.size, b) for b in range(256 * K)], dtype=np.uint16)
        out[f"tile_K{K}"] = tile
        out[f"win_K{K}"] = w
    np.savez_compressed(os.path.join(HERE, "windows.npz"), **out)


def ref_dequant(R, trellis_u16, suh, svh, K, mcg):
    """dequant_cpu's order of operations, with the reference's own scalar primitives."""
    kt_n, nt_n = trellis_u16.shape[:2]
    rows, cols = kt_n * 16, nt_n * 16
    M = np.zeros((rows, cols), dtype=np.float32)
    words = 16 * K
    for kt in range(kt_n):
        for nt in range(nt_n):
            tile = np.ascontiguousarray(trellis_u16[kt, nt])
            lane = [[0] * 8 for _ in range(32)]
            for l in range(32):
                for j in range(8):
                    start = (l * 8 + j + 257) * K - 16
                    win = R.ref_read_window(tile.ctypes.data, words, start)
                    lane[l][j] = R.ref_decode_codebook_bits(win, 1 if mcg else 2)
            for l in range(32):
                if l & 4:
                    continue
                row0, row2 = (l % 4) * 2, (l % 4) * 2 + 8
                col0, col4 = (l // 8) * 2, (l // 8) * 2 + 8
                own, peer = lane[l], lane[l + 4]
                for (r, c, j) in ((row0, col0, 0), (row0 + 1, col0, 1), (row2, col0, 2), (row2 + 1, col0, 3),
                                  (row0, col4, 4), (row0 + 1, col4, 5), (row2, col4, 6), (row2 + 1, col4, 7)):
                    M[kt * 16 + r, nt * 16 + c] = R.ref_half_bits_to_float(own[j])
                    M[kt * 16 + r, nt * 16 + c + 1] = R.ref_half_bits_to_float(peer[j])
    su = suh.astype(np.float32)
    sv = svh.astype(np.float32)
    W = np.zeros((rows, cols), dtype=np.float16)
    line = np.zeros(128, dtype=np.float32)
    for r0 in range(0, rows, 128):
        for c0 in range(0, cols, 128):
            for r in range(128):
                line[:] = M[r0 + r, c0:c0 + 128]
                R.ref_hadamard(line.ctypes.data, 128)
                M[r0 + r, c0:c0 + 128] = line * NORM
            for c in range(128):
                line[:] = M[r0:r0 + 128, c0 + c]
                R.ref_hadamard(line.ctypes.data, 128)
                v = (line * NORM) * su[r0:r0 + 128]
                v = v * sv[c0 + c]
                W[r0:r0 + 128, c0 + c] = v.astype(np.float16)
    return W.view(np.uint16)


def dequant(R):
    out = {}
    cases = [(2, True), (3, False), (4, True), (4, False), (5, True), (8, False)]
    for i, (K, mcg) in enumerate(cases):
        rng = np.random.default_rng(100 + i)
        k, n = 128, 256
        trellis = rng.integers(0, 65536, size=(k // 16, n // 16, 16 * K), dtype=np.uint16)
        suh = np.where(rng.random(k) < 0.5, -1.0, 1.0).astype(np.float16)
        svh = np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float16)
        W = ref_dequant(R, trellis, suh, svh, K, mcg)
        tag = f"K{K}_{'mcg' if mcg else 'mul1'}"
        out[f"trellis_{tag}"] = trellis
        out[f"suh_{tag}"] = suh
        out[f"svh_{tag}"] = svh
        out[f"W_{tag}"] = W
    np.savez_compressed(os.path.join(HERE, "dequant.npz"), **out)


if __name__ == "__main__":
    R = ref()
    codebooks(R)
    windows(R)
    dequant(R)
    print("golden vectors written to", HERE)
