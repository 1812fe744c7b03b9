"""Static per-architecture launch-shape table for the decode GEMV.

The reference autotunes its Triton GEMV at install time and persists the
winners per GPU name in configs/fused_tune.json (models/fused/kernels.py:
262-331).  Here the library's built-in per-shape rule (cfg all zero) is the
default and needs no warm-up; this table only overrides it where an offline
sweep on the target architecture (``python -m breeze_amd.tune``) measured a
better launch shape.  The table ships with the package
(``tune_<arch>.json``), is read once per process, and never changes at run
time, so a call stays capture-safe and reentrant.

Key: "<arch>|N|K|wfmt|epilogue|norm|M-bucket" (M-bucket = M rounded up to
1, 2, 4, 8, 16 or 32; larger M takes the 32 bucket), value: [depth, waves,
tiles, path] or [depth, waves, tiles, path, slices] as in bz_gemv_desc's
cfg fields.
"""

from __future__ import annotations

import json
import os
from pathlib import Path
from typing import Optional

import torch

PKG_DIR = Path(__file__).resolve().parent
_TABLES: dict[str, dict] = {}
_ARCH: dict[int, str] = {}

__all__ = ["arch_of", "m_bucket", "table_key", "lookup", "table_path"]


def table_path(arch: str) -> Path:
    return Path(os.environ.get("BZ_TUNE_TABLE", str(PKG_DIR / f"tune_{arch}.json")))


def arch_of(device: torch.device) -> str:
    """gfx name of the device ("gfx950"), cached per device index."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    a = _ARCH.get(idx)
    if a is None:
        a = torch.cuda.get_device_properties(idx).gcnArchName.split(":")[0]
        _ARCH[idx] = a
    return a


def m_bucket(M: int) -> int:
    for b in (1, 2, 4, 8, 16):
        if M <= b:
            return b
    return 32


def table_key(arch: str, N: int, K: int, wfmt: int, epilogue: int, norm: bool, M: int) -> str:
    return f"{arch}|{N}|{K}|{wfmt}|{epilogue}|{int(bool(norm))}|{m_bucket(M)}"


def _table(arch: str) -> dict:
    t = _TABLES.get(arch)
    if t is None:
        p = table_path(arch)
        t = json.loads(p.read_text()) if p.exists() else {}
        _TABLES[arch] = t
    return t


def lookup(device: torch.device, N: int, K: int, wfmt: int, epilogue: int, norm: bool, M: int) -> Optional[tuple]:
    """The table's launch shape for this GEMV, or None for the built-in rule."""
    arch = arch_of(device)
    cfg = _table(arch).get(table_key(arch, N, K, wfmt, epilogue, norm, M))
    return tuple(cfg) if cfg is not None else None
