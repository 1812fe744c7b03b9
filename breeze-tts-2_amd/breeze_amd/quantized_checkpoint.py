"""Pre-quantized checkpoints in this build's layouts.

The on-disk format follows models/quantized_checkpoint.py: a directory with
``quantized.safetensors`` (the model's state dict) and
``quant_manifest.json`` (format version, source, quant_config, tensor count,
byte total, and one entry per quantized module: kind, in/out features, group
size and buffer shapes).  The API has the same five entry points: describe,
save_quantized, install_shells, load_quantized_state, read_manifest.

This build's additions to the manifest and the loader:

* every int4 entry carries ``"layout"``, the tag of the bytes in its
  weight_int4 buffer (int4_linear.LAYOUT_TILED, "bz-int4-tiled16-v2", for
  the 16-row-block tiled layout of include/bz_gemv.h, or LAYOUT_ROWMAJOR,
  "bz-int4-rowmajor-evenlow-v1", for the row-major nibble matrix).  A
  row-major module of a tileable shape is re-tiled on its GPU after loading.
  An int4 entry without a tag is a checkpoint of the reference, whose
  weight_int4 holds tinygemm's architecture-specific repack
  (models/int4_linear.py:59); it is refused with an explanation rather than
  read as something it is not;
* the buffer shapes of every entry are checked against its features and
  group before any buffer is made, so a manifest that does not describe a
  buffer the GEMV can read fails at load time, not on the GPU;
* Fp8Linear modules are recorded too (kind "fp8"), with ``"layout"`` the
  tag of their weight_fp8 bytes (fp8_linear.LAYOUT_TILED,
  "bz-fp8-tiled16-v1", or LAYOUT_ROWMAJOR, "e4m3-rowmajor", the reference's
  [N, K] codes).  An fp8 entry without a tag is the reference's row-major
  buffer and is read as such; a row-major module of a tileable shape is
  re-tiled on its GPU after loading;
* ``convert_logical_int4`` turns the logical nibbles the reference's
  quantizer builds before its repack (odd k in the low nibble,
  models/int4_linear.py:57-58) into this build's row-major buffer.

The reference's Int8Linear (its text-embedding path) is not part of this
build; an ``int8`` entry is refused.
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path
from typing import Callable

import torch
from safetensors import safe_open
from safetensors.torch import save_file
from torch import nn

from . import fp8_linear as _f8
from .fp8_linear import FP8_DTYPE, Fp8Linear
from .int4_linear import LAYOUT_ROWMAJOR, LAYOUT_TILED, Int4Linear, layout_of, retile, tileable, tiled_shape

INT4_LAYOUT = LAYOUT_TILED
FORMAT_VERSION = 1
WEIGHTS_NAME = "quantized.safetensors"
MANIFEST_NAME = "quant_manifest.json"
# Embedding tables a caller may keep in host memory when offloading.
TEXT_EMBEDDING_PREFIXES = ("embed_text_tokens.", "text_encoder.embed_tokens.")

__all__ = [
    "FORMAT_VERSION",
    "WEIGHTS_NAME",
    "MANIFEST_NAME",
    "TEXT_EMBEDDING_PREFIXES",
    "INT4_LAYOUT",
    "describe",
    "save_quantized",
    "install_shells",
    "load_quantized_state",
    "read_manifest",
    "convert_logical_int4",
    "logical_int4",
]


@dataclass(frozen=True)
class _Kind:
    """How one quantized module class appears in the manifest."""

    name: str
    cls: type
    buffers: dict            # buffer name -> dtype
    attrs: tuple             # manifest keys copied to/from module attributes
    shapes: Callable         # spec -> {buffer: expected shape}


def _int4_shapes(spec: dict) -> dict:
    n, k, g = spec["out_features"], spec["in_features"], spec["group_size"]
    if g <= 0 or k % g:
        raise ValueError(f"group {g} does not divide in_features {k}")
    layout = spec.get("layout")
    if layout == LAYOUT_TILED:
        if not tileable(n, k, g):
            raise ValueError(f"a {n}x{k} weight with group {g} has no tiled layout")
        packed = list(tiled_shape(n, k))
    elif layout == LAYOUT_ROWMAJOR:
        packed = [n, k // 8]
    else:
        raise ValueError(
            f"int4 module stored in layout {layout!r}; this build reads {LAYOUT_TILED!r} and "
            f"{LAYOUT_ROWMAJOR!r}.  A checkpoint without a layout tag comes from the reference and holds "
            "tinygemm's architecture-specific packing: re-export it from the logical nibbles with "
            "convert_logical_int4")
    return {"weight_int4": packed, "scales_zeros": [k // g, n, 2]}


def _fp8_shapes(spec: dict) -> dict:
    n, k = spec["out_features"], spec["in_features"]
    layout = spec.get("layout", _f8.LAYOUT_ROWMAJOR)  # untagged: the reference's own [N, K] codes
    if layout == _f8.LAYOUT_TILED:
        if not _f8.tileable(n, k):
            raise ValueError(f"a {n}x{k} fp8 weight has no tiled layout")
        codes = list(_f8.tiled_shape(n, k))
    elif layout == _f8.LAYOUT_ROWMAJOR:
        codes = [n, k]
    else:
        raise ValueError(f"fp8 module stored in layout {layout!r}; this build reads {_f8.LAYOUT_TILED!r} and "
                         f"{_f8.LAYOUT_ROWMAJOR!r}")
    return {"weight_fp8": codes, "weight_scale": [1, n]}


_KINDS = (
    _Kind("int4", Int4Linear, {"weight_int4": torch.int32, "scales_zeros": torch.bfloat16},
          ("in_features", "out_features", "group_size"), _int4_shapes),
    _Kind("fp8", Fp8Linear, {"weight_fp8": FP8_DTYPE, "weight_scale": torch.float32},
          ("in_features", "out_features"), _fp8_shapes),
)
_BY_NAME = {k.name: k for k in _KINDS}


def _kind_of(module: nn.Module):
    return next((k for k in _KINDS if isinstance(module, k.cls)), None)


def describe(model: nn.Module) -> dict[str, dict]:
    """Manifest entries of every quantized module, keyed by module path."""
    entries: dict[str, dict] = {}
    for path, module in model.named_modules():
        kind = _kind_of(module)
        if kind is None:
            continue
        entry = {"kind": kind.name}
        if kind.name == "int4":
            entry["layout"] = layout_of(module.weight_int4, module.out_features, module.in_features)
        elif kind.name == "fp8":
            entry["layout"] = _f8.layout_of(module.weight_fp8, module.out_features, module.in_features)
        entry.update({a: int(getattr(module, a)) for a in kind.attrs})
        entry["shapes"] = {b: list(getattr(module, b).shape) for b in kind.buffers}
        entries[path] = entry
    return entries


def save_quantized(model: nn.Module, out_dir: Path, quant_config: dict, source: str) -> dict:
    """Write ``model``'s state dict and its manifest under ``out_dir``;
    returns the manifest."""
    target = Path(out_dir)
    target.mkdir(parents=True, exist_ok=True)
    # one private host copy per entry: safetensors refuses shared or strided storage
    tensors = {}
    for name, tensor in model.state_dict().items():
        tensors[name] = tensor.detach().to("cpu", copy=True).contiguous()
    save_file(tensors, str(target / WEIGHTS_NAME))
    manifest = dict(
        version=FORMAT_VERSION,
        source=source,
        quant_config=quant_config,
        modules=describe(model),
        tensor_count=len(tensors),
        bytes=sum(t.numel() * t.element_size() for t in tensors.values()),
    )
    with open(target / MANIFEST_NAME, "w") as fh:
        json.dump(manifest, fh, indent=2)
        fh.write("\n")
    return manifest


def _shell(path: str, spec: dict, device) -> nn.Module:
    """An empty module of the entry's kind, buffers allocated on ``device``
    with the shapes the manifest records, after checking those shapes."""
    kind = _BY_NAME.get(spec.get("kind"))
    if kind is None:
        raise ValueError(f"{path}: module kind {spec.get('kind')!r} is not part of this build")
    want = kind.shapes(spec)
    have = {b: list(s) for b, s in spec.get("shapes", {}).items()}
    if have != want:
        raise ValueError(f"{path}: manifest buffer shapes {have} do not match the module's {want}")
    module = kind.cls.__new__(kind.cls)
    nn.Module.__init__(module)
    for attr in kind.attrs:
        setattr(module, attr, int(spec[attr]))
    for name, dtype in kind.buffers.items():
        module.register_buffer(name, torch.empty(want[name], dtype=dtype, device=device))
    return module


def install_shells(model: nn.Module, manifest: dict, device) -> int:
    """Put an empty quantized module at every path the manifest lists, so
    that the state dict has somewhere to land.  Returns how many."""
    shells = {path: _shell(path, spec, device) for path, spec in manifest["modules"].items()}
    for path, shell in shells.items():
        parent_path, _, attr = path.rpartition(".")
        parent = model.get_submodule(parent_path) if parent_path else model
        setattr(parent, attr, shell)
    return len(shells)


def load_quantized_state(model: nn.Module, out_dir: Path, device, host_prefixes: tuple[str, ...] = ()) -> dict:
    """Load the checkpoint into ``model`` (shells installed), tensors on
    ``device`` except those whose name starts with one of ``host_prefixes``,
    which stay in host memory.  Row-major int4 and fp8 modules of a tileable
    shape are re-tiled when they land on a GPU.  Returns counts and a few names of
    missing and unexpected keys."""
    state = {}
    with safe_open(str(Path(out_dir) / WEIGHTS_NAME), framework="pt", device="cpu") as reader:
        for name in reader.keys():
            where = "cpu" if host_prefixes and name.startswith(tuple(host_prefixes)) else device
            state[name] = reader.get_tensor(name).to(where)
    result = model.load_state_dict(state, strict=False, assign=True)
    for module in model.modules():
        if isinstance(module, Int4Linear) and module.weight_int4.is_cuda:
            retile(module)
        elif isinstance(module, Fp8Linear) and module.weight_fp8.is_cuda:
            _f8.retile(module)
    missing, unexpected = list(result.missing_keys), list(result.unexpected_keys)
    return {
        "loaded": len(state),
        "missing": len(missing),
        "unexpected": len(unexpected),
        "missing_sample": missing[:5],
        "unexpected_sample": unexpected[:5],
    }


def read_manifest(out_dir: Path) -> dict:
    """The manifest of a checkpoint directory, after checking its version."""
    with open(Path(out_dir) / MANIFEST_NAME) as fh:
        manifest = json.load(fh)
    version = manifest.get("version")
    if version != FORMAT_VERSION:
        raise ValueError(f"unsupported checkpoint version {version!r} (this build reads {FORMAT_VERSION})")
    if not isinstance(manifest.get("modules"), dict):
        raise ValueError("checkpoint manifest has no module table")
    return manifest


def convert_logical_int4(packed_odd_low: torch.Tensor, scales_zeros: torch.Tensor, group_size: int = 128):
    """The reference quantizer's logical nibbles -> this build's row-major
    int4 buffers.

    packed_odd_low: uint8 [N, K/2], byte j of row n = q[n, 2j+1] | q[n, 2j] << 4
    (models/int4_linear.py:57-58).  Returns (weight_int4 int32 [N, K/8] with
    even k in the low nibble, scales_zeros unchanged, bf16 [K/group, N, 2]).
    Pure integer nibble swap: w_eff is identical bit for bit.  A module
    holding the result reads it as LAYOUT_ROWMAJOR; int4_linear.retile moves
    it to the tiled layout on a GPU."""
    if packed_odd_low.dtype != torch.uint8 or packed_odd_low.dim() != 2:
        raise ValueError("packed_odd_low must be a uint8 [N, K/2] tensor")
    N, half = packed_odd_low.shape
    K = 2 * half
    if K % group_size or half % 4:
        raise ValueError(f"K = {K} must be a multiple of the group {group_size} and of 8")
    if tuple(scales_zeros.shape) != (K // group_size, N, 2):
        raise ValueError(f"scales_zeros shape {tuple(scales_zeros.shape)} != {(K // group_size, N, 2)}")
    swapped = ((packed_odd_low & 0x0F) << 4) | (packed_odd_low >> 4)
    return swapped.contiguous().view(torch.int32), scales_zeros.to(torch.bfloat16).contiguous()


def logical_int4(weight_int4: torch.Tensor) -> torch.Tensor:
    """Inverse of convert_logical_int4's nibble swap: a row-major weight_int4
    -> the reference's logical uint8 [N, K/2] (odd k in the low nibble)."""
    b = weight_int4.contiguous().view(torch.uint8)
    return (((b & 0x0F) << 4) | (b >> 4)).contiguous()
