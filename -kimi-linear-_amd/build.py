"""Build ``libkda_hip.so`` (the gfx950 KDA kernels + C ABI) in-tree with hipcc.

Usage: ``python -kimi-linear-_amd/build.py`` or ``build_native()`` from Python.
The library lands next to this file, where ``_native.py`` loads it from.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
LIB_PATH = PKG_DIR / "libkda_hip.so"
BUILD_DIR = PKG_DIR / "_build"

SOURCES = ["kda_api.hip", "kda_recurrent.hip", "kda_chunkwise.hip", "kda_chunkwise_bwd.hip", "kda_layer_ops.hip",
           "kda_layer_bwd.hip", "kda_long.hip", "kda_ckpt_fp32.hip"]

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 in the device code.
HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found: a ROCm toolchain is required to build libkda_hip.so")
    return exe


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{proc.stdout}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def build_native(verbose: bool = False) -> Path:
    """Compile every source for gfx950 and link the shared library."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    incs = [f"-I{INCLUDE}", f"-I{CSRC}"]

    def compile_one(src: str) -> Path:
        obj = BUILD_DIR / (Path(src).stem + ".o")
        cmd = [hipcc, *HIPCC_FLAGS, *incs, "-c", str(CSRC / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd))
        _run(cmd)
        return obj

    workers = max(1, min(len(SOURCES), int(os.environ.get("MAX_JOBS", "4"))))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(compile_one, SOURCES))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd))
    _run(cmd)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build_native(verbose="-v" in sys.argv))
