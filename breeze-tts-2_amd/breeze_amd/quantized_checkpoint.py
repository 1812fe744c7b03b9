"""Save and load an already-quantized checkpoint in this build's layouts
(mirrors models/quantized_checkpoint.py).

Same files and API as the reference: ``quantized.safetensors`` holds the
state dict, ``quant_manifest.json`` records every quantized module with its
buffer shapes so ``install_shells`` can rebuild empty modules (on any device,
``meta`` included) for ``load_quantized_state`` to fill, and
``read_manifest`` checks the format version.

What this build adds:

* every int4 entry carries ``"layout"``: ``int4_linear.LAYOUT``
  ("bz-int4-rowmajor-evenlow-v1": weight_int4 is the row-major nibble matrix
  [N, K/2] viewed as int32 [N, K/8], even k in the low nibble; scales_zeros
  bf16 [K/group, N, 2] unchanged).  An int4 entry without that tag -- a
  checkpoint written by the reference, whose weight_int4 is tinygemm's
  architecture-specific tile layout (models/int4_linear.py:59,
  validate_sm86.py:3-7) -- is refused with an explanation instead of being
  read as something it is not;
* ``convert_logical_int4`` turns the logical nibble form the reference's
  quantizer builds before its tinygemm repack (byte j of row n = q[n, 2j+1] |
  q[n, 2j] << 4, odd k in the low nibble, models/int4_linear.py:57-58) plus
  its scales_zeros into this layout, so a reference export that keeps the
  logical nibbles converts without re-quantizing;
* Fp8Linear modules are recorded too (``"kind": "fp8"``, buffers weight_fp8
  e4m3fn [N, K] and weight_scale fp32 [1, N]); the reference quantizes fp8 at
  load time instead.

The reference's Int8Linear (text-embedding path) is not part of this build:
an ``int8`` entry is refused by ``install_shells``.
"""

from __future__ import annotations

import json
from pathlib import Path

import torch
from safetensors.torch import load_file, save_file
from torch import nn

from .fp8_linear import FP8_DTYPE, Fp8Linear
from .int4_linear import LAYOUT as INT4_LAYOUT
from .int4_linear import Int4Linear

FORMAT_VERSION = 1
WEIGHTS_NAME = "quantized.safetensors"
MANIFEST_NAME = "quant_manifest.json"
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


def describe(model: nn.Module) -> dict[str, dict]:
    """Every quantized module with what install_shells needs to rebuild it
    (models/quantized_checkpoint.py:35-63, plus the int4 layout tag)."""
    described: dict[str, dict] = {}
    for path, module in model.named_modules():
        if isinstance(module, Int4Linear):
            described[path] = {
                "kind": "int4",
                "layout": INT4_LAYOUT,
                "in_features": module.in_features,
                "out_features": module.out_features,
                "group_size": module.group_size,
                "shapes": {
                    "weight_int4": list(module.weight_int4.shape),
                    "scales_zeros": list(module.scales_zeros.shape),
                },
            }
        elif isinstance(module, Fp8Linear):
            described[path] = {
                "kind": "fp8",
                "in_features": module.in_features,
                "out_features": module.out_features,
                "shapes": {
                    "weight_fp8": list(module.weight_fp8.shape),
                    "weight_scale": list(module.weight_scale.shape),
                },
            }
    return described


def save_quantized(model: nn.Module, out_dir: Path, quant_config: dict, source: str) -> dict:
    """Write the state dict and the manifest (models/quantized_checkpoint.py:66-91)."""
    out_dir = Path(out_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    modules = describe(model)
    # safetensors wants contiguous tensors without shared storage
    state = {key: value.detach().cpu().contiguous().clone() for key, value in model.state_dict().items()}
    save_file(state, str(out_dir / WEIGHTS_NAME))
    manifest = {
        "version": FORMAT_VERSION,
        "source": source,
        "quant_config": quant_config,
        "modules": modules,
        "tensor_count": len(state),
        "bytes": sum(v.numel() * v.element_size() for v in state.values()),
    }
    (out_dir / MANIFEST_NAME).write_text(json.dumps(manifest, indent=2) + "\n")
    return manifest


def _empty_int4(spec: dict, device) -> Int4Linear:
    layout = spec.get("layout")
    if layout != INT4_LAYOUT:
        raise ValueError(
            f"int4 module stored in layout {layout!r}, this build reads {INT4_LAYOUT!r}: a checkpoint "
            "written by the reference holds tinygemm's architecture-specific packing; re-export it "
            "from the logical nibbles with convert_logical_int4"
        )
    module = Int4Linear.__new__(Int4Linear)
    nn.Module.__init__(module)
    module.in_features = spec["in_features"]
    module.out_features = spec["out_features"]
    module.group_size = spec["group_size"]
    module.register_buffer("weight_int4",
                           torch.empty(spec["shapes"]["weight_int4"], dtype=torch.int32, device=device))
    module.register_buffer("scales_zeros",
                           torch.empty(spec["shapes"]["scales_zeros"], dtype=torch.bfloat16, device=device))
    return module


def _empty_fp8(spec: dict, device) -> Fp8Linear:
    module = Fp8Linear.__new__(Fp8Linear)
    nn.Module.__init__(module)
    module.in_features = spec["in_features"]
    module.out_features = spec["out_features"]
    module.register_buffer("weight_fp8", torch.empty(spec["shapes"]["weight_fp8"], dtype=FP8_DTYPE, device=device))
    module.register_buffer("weight_scale",
                           torch.empty(spec["shapes"]["weight_scale"], dtype=torch.float32, device=device))
    return module


def _set_submodule(root: nn.Module, path: str, replacement: nn.Module) -> None:
    parts = path.split(".")
    parent = root
    for part in parts[:-1]:
        parent = getattr(parent, part)
    setattr(parent, parts[-1], replacement)


def install_shells(model: nn.Module, manifest: dict, device) -> int:
    """Empty quantized modules where the manifest says, so the state dict has
    somewhere to land (models/quantized_checkpoint.py:137-142)."""
    builders = {"int4": _empty_int4, "fp8": _empty_fp8}
    for path, spec in manifest["modules"].items():
        builder = builders.get(spec["kind"])
        if builder is None:
            raise ValueError(f"{path}: module kind {spec['kind']!r} is not part of this build")
        _set_submodule(model, path, builder(spec, device))
    return len(manifest["modules"])


def load_quantized_state(model: nn.Module, out_dir: Path, device, host_prefixes: tuple[str, ...] = ()) -> dict:
    """Fill installed shells from the checkpoint; tensors under
    ``host_prefixes`` stay in host memory (models/quantized_checkpoint.py:145-175)."""
    out_dir = Path(out_dir)
    if host_prefixes:
        from safetensors import safe_open

        state = {}
        with safe_open(str(out_dir / WEIGHTS_NAME), framework="pt") as handle:
            for key in handle.keys():  # noqa: SIM118 - safetensors API
                target = "cpu" if key.startswith(host_prefixes) else str(device)
                state[key] = handle.get_tensor(key).to(target)
    else:
        state = load_file(str(out_dir / WEIGHTS_NAME), device=str(device))
    missing, unexpected = model.load_state_dict(state, strict=False, assign=True)
    return {
        "loaded": len(state),
        "missing": len(missing),
        "unexpected": len(unexpected),
        "missing_sample": list(missing)[:5],
        "unexpected_sample": list(unexpected)[:5],
    }


def read_manifest(out_dir: Path) -> dict:
    manifest = json.loads((Path(out_dir) / MANIFEST_NAME).read_text())
    if manifest.get("version") != FORMAT_VERSION:
        raise ValueError(f"unsupported checkpoint version {manifest.get('version')!r}")
    return manifest


def convert_logical_int4(packed_odd_low: torch.Tensor, scales_zeros: torch.Tensor, group_size: int = 128):
    """The reference quantizer's logical nibbles -> this build's int4 buffers.

    packed_odd_low: uint8 [N, K/2], byte j of row n = q[n, 2j+1] | q[n, 2j] << 4
    (models/int4_linear.py:57-58).  Returns (weight_int4 int32 [N, K/8] with
    even k in the low nibble, scales_zeros unchanged, bf16 [K/group, N, 2]).
    Pure integer nibble swap: w_eff is identical bit for bit."""
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
    """Inverse of convert_logical_int4's nibble swap: this build's weight_int4
    -> the reference's logical uint8 [N, K/2] (odd k in the low nibble)."""
    b = weight_int4.contiguous().view(torch.uint8)
    return (((b & 0x0F) << 4) | (b >> 4)).contiguous()
