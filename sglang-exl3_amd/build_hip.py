"""Build the gfx950 HIP library libsglang_exl3_amd.so in-tree.

Compiles every csrc/*.hip (the GEMV instantiation unit once per bit width)
with hipcc for gfx950 and links one shared library into
sglang_exl3/_lib/.  Run directly (python build_hip.py) or through
__graft_entry__.build().
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIBDIR = os.path.join(HERE, "sglang_exl3", "_lib")
LIBNAME = "libsglang_exl3_amd.so"
ARCH = os.environ.get("EXL3_OFFLOAD_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
COMMON = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # packed-fp32 instructions stay off (some packed forms have given silent wrong results on these boxes)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result", "-Wno-pass-failed",
]
# bit widths the GEMV family is instantiated for
GEMV_KS = (1, 2, 3, 4, 5, 6, 7, 8)


def _units():
    units = []
    for fn in sorted(os.listdir(CSRC)):
        if not fn.endswith(".hip"):
            continue
        src = os.path.join(CSRC, fn)
        stem = fn[:-4]
        if stem.endswith("_inst"):
            for K in GEMV_KS:
                units.append((src, os.path.join(BUILD, f"{stem}_K{K}.o"), [f"-DEXL3_K={K}"]))
        else:
            units.append((src, os.path.join(BUILD, f"{stem}.o"), []))
    return units


def _headers_mtime() -> float:
    hs = [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")]
    hs.append(os.path.join(HERE, "..", "include", "sglang_exl3_amd.h"))
    return max(os.path.getmtime(h) for h in hs if os.path.exists(h))


def _compile(unit, force: bool):
    src, obj, extra = unit
    if not force and os.path.exists(obj):
        if os.path.getmtime(obj) >= max(os.path.getmtime(src), _headers_mtime()):
            return obj, "cached"
    cmd = [HIPCC, *COMMON, *extra, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {os.path.basename(src)} {extra}:\n{r.stderr[-6000:]}")
    return obj, "built"


def build(force: bool = False, jobs: int | None = None) -> str:
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    units = _units()
    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = [o for o, _ in ex.map(lambda u: _compile(u, force), units)]
    out = os.path.join(LIBDIR, LIBNAME)
    tmp = out + ".tmp"
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-6000:]}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    path = build(force="--force" in sys.argv)
    print(path)
