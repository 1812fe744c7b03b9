"""Weight-only int4 Linear for bandwidth-bound decode, on MI355X.

Drop-in for models/int4_linear.py: same names (GROUP_SIZE, MIN_QUANT_BYTES,
DEFAULT_TARGET_NAMES, quantize_int4, Int4Linear, quantize_module_int4), same
constructor arguments, forward() contract, buffer names/dtypes, error
messages and stats dict.

What changes is the packed layout held in ``weight_int4`` and the kernel.
The reference hands its nibbles to torch's tinygemm repack
(models/int4_linear.py:59), an architecture-specific opaque tile format.
Here ``weight_int4`` holds one of this build's two documented layouts
(include/bz_gemv.h), told apart by its shape:

  tiled (LAYOUT_TILED, whenever out_features % 16 == 0, in_features % 128
  == 0 and group 128 -- every decode shape of the model): int32
      [N/16, chunk/4], the bytes of BZ_W_INT4_TILED: per block of 16 output
      rows, K/128 tiles of 1 KiB (16 rows x 128 k, even k in the low nibble)
      followed by the block's (s, z) pairs; read by the streaming GEMV path;
  row-major (LAYOUT_ROWMAJOR, any other shape or group): int32 [N, K/8],
      the bytes of uint8 [N, K/2] with byte j of row n = q[n, 2j] |
      q[n, 2j+1] << 4 (models/fused/kernels.py:149).

    scales_zeros: bf16 [K/group, N, 2] = (s, z), exactly as the reference
                  stores it (models/int4_linear.py:61-63), in both cases
    w_eff[n, k] = (q[n, k] - 8) * s[k/group, n] + z[k/group, n]

The tiled layout repeats the (s, z) pairs inside weight_int4 (6.25% of the
packed bytes) so that every workgroup of the GEMV streams one contiguous
chunk; scales_zeros stays the reference's buffer for checkpoints and
inspection.  Quantization itself is the reference's min/max scheme
(models/int4_linear.py:47-54), run by a HIP kernel that reproduces its float32
steps bit for bit.
"""

from __future__ import annotations

import torch
from torch import nn

from ._swap import swap_linears
from .gemv import (W_INT4_TILED, W_INT4_ZP, dequant_matmul, gemv_traceable, pack_tiled, quantize_int4_device,
                   tiled_bytes)

GROUP_SIZE = 128

# Below this, layers are cache-resident and launch-bound rather than
# bandwidth-bound (models/int4_linear.py:39-42).
MIN_QUANT_BYTES = 8 * 1024 * 1024

DEFAULT_TARGET_NAMES = ("gate_proj", "up_proj", "down_proj")

# Above this many rows a call is a prefill rather than a decode step: a tiled
# weight is then decoded to bf16 in bounded row chunks and multiplied by the
# library GEMM, instead of being streamed once per 32 rows by the GEMV.
PREFILL_ROWS = 32

# Tags recorded by the checkpoint manifest for the two packed layouts.
LAYOUT_TILED = "bz-int4-tiled16-v2"
LAYOUT_ROWMAJOR = "bz-int4-rowmajor-evenlow-v1"
LAYOUT = LAYOUT_TILED


def tileable(out_features: int, in_features: int, group_size: int) -> bool:
    """Whether a weight of this shape is stored in the tiled layout."""
    return out_features % 16 == 0 and in_features % 128 == 0 and group_size == 128


def tiled_shape(out_features: int, in_features: int) -> tuple[int, int]:
    """int32 shape of a tiled weight_int4: [N/16, bytes per 16-row block / 4]."""
    return out_features // 16, tiled_bytes(W_INT4_TILED, 16, in_features) // 4


def layout_of(weight_int4: torch.Tensor, out_features: int, in_features: int) -> str:
    """The layout a weight_int4 buffer holds, from its shape."""
    if tuple(weight_int4.shape) == (out_features, in_features // 8):
        return LAYOUT_ROWMAJOR
    return LAYOUT_TILED


def _check_group(in_features: int, group_size: int) -> None:
    if in_features % group_size:
        raise ValueError(f"in_features {in_features} not divisible by group {group_size}")
    if group_size < 32 or group_size & (group_size - 1):
        raise ValueError(f"group {group_size} unsupported: must be a power of two >= 32")


def quantize_int4(weight: torch.Tensor, group_size: int = GROUP_SIZE, symmetric: bool = False):
    """Group-wise int4 quantisation into this build's layout.

    Asymmetric (default, models/int4_linear.py:47-64): per group lo = min,
    s = max((max - lo)/15, 1e-8), q = clamp(rne((w - lo)/s), 0, 15),
    z = lo + 8 s.  symmetric=True: s = absmax/7, q = clamp(rne(w/s) + 8, 0, 15),
    z = 0.  Returns (weight_int4 int32, tiled [N/16, chunk/4] when the shape
    is tileable else row-major [N, K/8]; scales_zeros bf16 [K/group, N, 2]) on
    the device the weight lives on (a CPU weight is quantized on the current
    GPU and the result moved back).
    """
    out_features, in_features = weight.shape
    _check_group(in_features, group_size)
    packed, scales_zeros, _ = quantize_int4_device(weight, group_size, symmetric, W_INT4_ZP)
    if tileable(out_features, in_features, group_size):
        tiled = pack_tiled(W_INT4_ZP, packed, in_features, W_INT4_TILED, sc0=scales_zeros)
        inner = tiled.view(torch.int32).view(*tiled_shape(out_features, in_features))
    else:
        inner = packed.view(torch.int32)
    if weight.device.type != "cuda":
        inner, scales_zeros = inner.to(weight.device), scales_zeros.to(weight.device)
    return inner.contiguous(), scales_zeros.contiguous()


def retile(module: "Int4Linear") -> bool:
    """Convert a row-major Int4Linear (e.g. loaded from a checkpoint written
    in LAYOUT_ROWMAJOR) to the tiled layout in place, on its GPU.  Returns
    whether it changed."""
    if layout_of(module.weight_int4, module.out_features, module.in_features) != LAYOUT_ROWMAJOR:
        return False
    if not tileable(module.out_features, module.in_features, module.group_size):
        return False
    tiled = pack_tiled(W_INT4_ZP, module.weight_int4.view(torch.uint8), module.in_features, W_INT4_TILED,
                       sc0=module.scales_zeros)
    module.weight_int4 = tiled.view(torch.int32).view(*tiled_shape(module.out_features, module.in_features))
    return True


class Int4Linear(nn.Module):
    """Drop-in replacement for a bias-free nn.Linear using int4 weights."""

    def __init__(
        self,
        linear: nn.Linear,
        group_size: int = GROUP_SIZE,
        device: torch.device | str | None = None,
    ) -> None:
        super().__init__()
        if linear.bias is not None:
            raise ValueError("Int4Linear expects a bias-free Linear")
        # A CPU-resident model can be quantized one layer at a time on the GPU
        # by passing device=; only the packed form stays.
        weight = linear.weight.data if device is None else linear.weight.data.to(device)
        self.out_features, self.in_features = (int(d) for d in weight.shape)
        self.group_size = group_size
        _check_group(self.in_features, group_size)
        packed, scales_zeros = quantize_int4(weight, group_size)
        self.register_buffer("weight_int4", packed)
        self.register_buffer("scales_zeros", scales_zeros)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shape = x.shape
        flat = x.reshape(-1, shape[-1])
        if layout_of(self.weight_int4, self.out_features, self.in_features) == LAYOUT_TILED:
            wfmt, sc0 = W_INT4_TILED, None
            if flat.shape[0] > PREFILL_ROWS and not torch.compiler.is_compiling():
                out = dequant_matmul(flat, self.weight_int4, W_INT4_TILED, self.out_features, self.in_features)
                return out.to(x.dtype).reshape(*shape[:-1], self.out_features)
        else:
            wfmt, sc0 = W_INT4_ZP, self.scales_zeros
        out = gemv_traceable(
            flat.to(torch.bfloat16),
            self.weight_int4,
            wfmt,
            self.out_features,
            sc0=sc0,
            group=self.group_size,
        )
        return out.to(x.dtype).reshape(*shape[:-1], self.out_features)

    def extra_repr(self) -> str:
        return (
            f"in_features={self.in_features}, out_features={self.out_features}, "
            f"int4=True, group={self.group_size}"
        )


def quantize_module_int4(
    root: nn.Module,
    *,
    target_names: tuple[str, ...] = DEFAULT_TARGET_NAMES,
    min_bytes: int = MIN_QUANT_BYTES,
    device: torch.device | str | None = None,
    group_size: int = GROUP_SIZE,
) -> dict[str, int]:
    """Swap qualifying Linear layers under ``root`` for int4 equivalents
    (models/int4_linear.py:118-164).  A layer that cannot be packed is left
    untouched and counted as ``skipped_unsupported``; the bf16 original of a
    converted layer is released at once.  Saved bytes: int4 keeps a quarter
    of a bf16 weight."""
    st = swap_linears(
        root,
        target_names,
        min_bytes,
        build=lambda lin: Int4Linear(lin, group_size=group_size, device=device),
        saved_bytes=lambda nbytes: nbytes - nbytes // 4,
        tolerate_errors=True,
        drop_original=True,
    )
    return {
        "converted": st.converted,
        "skipped_below_threshold": st.small,
        "skipped_unsupported": st.unsupported,
        "weight_bytes_saved": st.saved,
    }
