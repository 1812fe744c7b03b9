"""Compile libbzgemv.so (the gfx950 kernels + C ABI) in-tree.

    python -m breeze_amd.build          (from breeze-tts-2_amd/)

The library is written next to this file so that it travels with the source
tree; nothing is installed.  Every .hip source is compiled separately (in
parallel) and linked with hipcc.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
SRC_DIR = PKG_DIR.parent / "csrc"
INCLUDE_DIR = PKG_DIR.parents[1] / "include"
LIB_NAME = "libbzgemv.so"
LIB_PATH = PKG_DIR / LIB_NAME
ARCH = "gfx950"

# Packed-fp32 instructions stay disabled: hipcc would otherwise emit
# v_pk_{add,mul,fma}_f32 from ordinary float code.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE_DIR}",
    f"-I{SRC_DIR}",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the gfx950 kernels cannot be built")


def sources() -> list[Path]:
    return sorted(SRC_DIR.glob("*.hip"))


def build(verbose: bool = False) -> Path:
    """Compile every HIP source for gfx950 and link LIB_PATH.  Always
    recompiles (this is the build check)."""
    hipcc = _hipcc()
    obj_dir = PKG_DIR / "_build"
    obj_dir.mkdir(exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {SRC_DIR}")

    def compile_one(src: Path) -> Path:
        obj = obj_dir / (src.stem + ".o")
        cmd = [hipcc, *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
        return obj

    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as pool:
        objs = list(pool.map(compile_one, srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
