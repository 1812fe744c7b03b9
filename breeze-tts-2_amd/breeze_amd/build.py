"""Compile libbzgemv.so (the gfx950 kernels + C ABI) in-tree.

    python -m breeze_amd.build          (from breeze-tts-2_amd/)

The library is written next to this file so that it travels with the source
tree; nothing is installed.  Every .hip source is compiled separately (in
parallel) and linked with hipcc.
"""

from __future__ import annotations

import os
import re
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
    # leading scalar kernel arguments arrive in SGPRs at wave launch (kernarg
    # preloading; the streaming kernels pass their hot fields that way)
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    f"-I{INCLUDE_DIR}",
    f"-I{SRC_DIR}",
]


# Kernels of the decode paths that must not use scratch (private memory): a
# spilled or dynamically indexed register array costs a memory round trip per
# access.  Patterns over the mangled names; the attention kernel's bf16-cache
# instances with D <= 256 (attn_kernel<DL = 1, 2, 4, GM, F32C = false, ...>)
# are covered, its fp32-cache and D = 512 instances are allowed scratch.
NO_SCRATCH = (r"gemv_persist", r"gemv_mfma", r"gemv_i8mma", r"gemv_tile", r"gemv_stream", r"gemv_wide", r"gemv_panel",
              r"head_f32", r"qkv_rope_cache",
              r"attn_kernelILi[124]ELi\d+ELb0E")


def kernel_resources(remarks: str) -> list[tuple[str, int, int]]:
    """(kernel, VGPRs, scratch bytes per lane) from hipcc's
    -Rpass-analysis=kernel-resource-usage remarks."""
    out, name, vgpr = [], None, 0
    for line in remarks.splitlines():
        if "remark:" not in line:
            continue
        body = line.split("remark:", 1)[1].strip()
        body = body.split(" [-Rpass", 1)[0]
        if body.startswith("Function Name:"):
            name, vgpr = body.split(":", 1)[1].strip(), 0
        elif body.startswith("VGPRs:") and name:
            vgpr = int(body.split(":")[1].split()[0])
        elif body.startswith("ScratchSize") and name:
            out.append((name, vgpr, int(body.split(":")[1].split()[0])))
            name = None
    return out


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

    def compile_one(src: Path) -> tuple[Path, list]:
        obj = obj_dir / (src.stem + ".o")
        cmd = [hipcc, *HIP_FLAGS, "-Rpass-analysis=kernel-resource-usage", "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
        return obj, kernel_resources(res.stderr)

    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as pool:
        done = list(pool.map(compile_one, srcs))
    objs = [o for o, _ in done]
    kernels = sorted({k for _, ks in done for k in ks})
    (obj_dir / "kernel_resources.txt").write_text(
        "".join(f"{vg:4d} vgpr {sc:6d} scratch  {name}\n" for name, vg, sc in kernels))
    spilled = [name for name, _, sc in kernels if sc and any(re.search(t, name) for t in NO_SCRATCH)]
    if spilled:
        raise RuntimeError("decode kernels using scratch memory:\n  " + "\n  ".join(spilled))
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
