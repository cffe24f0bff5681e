"""Build the native encoder library (``libexl3_hip.so``) in-tree with hipcc.

Replaces the reference's JIT build of its SYCL extension
(exl3_quant/xpu_quantizer.py:65-98, ``build_quantize_extension``): here the
library is a plain C-ABI shared object compiled ahead of time for gfx950 and
loaded with ctypes, so the GPU box runs the prebuilt file without a compiler.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import time
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_ROOT = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
SOURCES = [CSRC / "exl3_encoder.hip", CSRC / "exl3_layer.hip"]
HEADERS = [CSRC / "exl3_layout.h", CSRC / "exl3_errors.h", REPO_ROOT / "include" / "exl3_encoder.h",
           REPO_ROOT / "include" / "exl3_layer.h"]
LIB_PATH = PKG_DIR / "libexl3_hip.so"
OFFLOAD_ARCH = os.environ.get("EXL3_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # fp16 arithmetic must round exactly as written: no contraction of
    # separate multiplies and adds, no fast-math.
    "-ffp-contract=off",
    "-fno-fast-math",
    # Packed-fp32 instructions are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]

_LAST_BUILD_SECONDS = 0.0


def hipcc_path() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise FileNotFoundError("hipcc not found (set HIPCC or install ROCm)")


def needs_rebuild() -> bool:
    if not LIB_PATH.exists():
        return True
    mtime = LIB_PATH.stat().st_mtime
    return any(p.stat().st_mtime > mtime for p in SOURCES + HEADERS)


def build_native(force: bool = True, verbose: bool = False) -> Path:
    """Compile ``libexl3_hip.so`` for gfx950. ``force=False`` skips an
    up-to-date build."""
    global _LAST_BUILD_SECONDS
    if not force and not needs_rebuild():
        return LIB_PATH
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc_path(), *HIPCC_FLAGS, "-o", str(tmp), *map(str, SOURCES)]
    t0 = time.perf_counter()
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + " ".join(cmd) + "\n" + res.stdout + res.stderr)
    if verbose and (res.stdout or res.stderr):
        print(res.stdout + res.stderr)
    os.replace(tmp, LIB_PATH)
    _LAST_BUILD_SECONDS = time.perf_counter() - t0
    return LIB_PATH


def last_build_seconds() -> float:
    return _LAST_BUILD_SECONDS


if __name__ == "__main__":
    print(build_native(force=True, verbose=True))
