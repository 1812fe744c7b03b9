"""Weight-only int4 Linear for bandwidth-bound decode, on MI355X.

Drop-in for models/int4_linear.py: same names (GROUP_SIZE, MIN_QUANT_BYTES,
DEFAULT_TARGET_NAMES, quantize_int4, Int4Linear, quantize_module_int4), same
constructor arguments, forward() contract, buffer names/dtypes, error
messages and stats dict.

What changes is the packed layout held in ``weight_int4`` and the kernel.
The reference hands its nibbles to torch's tinygemm repack
(models/int4_linear.py:59), an architecture-specific opaque tile format.
Here ``weight_int4`` is the plain row-major nibble matrix, viewed as int32:

    weight_int4 : int32 [N, K/8]  (the bytes of uint8 [N, K/2])
                  byte j of row n = q[n, 2j] | q[n, 2j+1] << 4
                  (even k in the low nibble: models/fused/kernels.py:149)
    scales_zeros: bf16 [K/group, N, 2] = (s, z), exactly as the reference
                  stores it (models/int4_linear.py:61-63)
    w_eff[n, k] = (q[n, k] - 8) * s[k/group, n] + z[k/group, n]

The GEMV streams those rows once per call with 16-byte loads; see
csrc/bz_gemv.hip.  Quantization itself is the reference's min/max scheme
(models/int4_linear.py:47-54), run by a HIP kernel that reproduces its float32
steps bit for bit.
"""

from __future__ import annotations

import torch
from torch import nn

from ._swap import swap_linears
from .gemv import W_INT4_ZP, gemv_traceable, quantize_int4_device

GROUP_SIZE = 128

# Below this, layers are cache-resident and launch-bound rather than
# bandwidth-bound (models/int4_linear.py:39-42).
MIN_QUANT_BYTES = 8 * 1024 * 1024

DEFAULT_TARGET_NAMES = ("gate_proj", "up_proj", "down_proj")

# Tag recorded by the checkpoint manifest for this packed layout.
LAYOUT = "bz-int4-rowmajor-evenlow-v1"


def _check_group(in_features: int, group_size: int) -> None:
    if in_features % group_size:
        raise ValueError(f"in_features {in_features} not divisible by group {group_size}")
    if group_size < 32 or group_size & (group_size - 1):
        raise ValueError(f"group {group_size} unsupported: must be a power of two >= 32")


def quantize_int4(weight: torch.Tensor, group_size: int = GROUP_SIZE, symmetric: bool = False):
    """Group-wise int4 quantisation into the row-major layout.

    Asymmetric (default, models/int4_linear.py:47-64): per group lo = min,
    s = max((max - lo)/15, 1e-8), q = clamp(rne((w - lo)/s), 0, 15),
    z = lo + 8 s.  symmetric=True: s = absmax/7, q = clamp(rne(w/s) + 8, 0, 15),
    z = 0.  Returns (weight_int4 int32 [N, K/8], scales_zeros bf16
    [K/group, N, 2]) on the device the weight lives on (a CPU weight is
    quantized on the current GPU and the result moved back).
    """
    out_features, in_features = weight.shape
    _check_group(in_features, group_size)
    packed, scales_zeros, _ = quantize_int4_device(weight, group_size, symmetric, W_INT4_ZP)
    inner = packed.view(torch.int32)
    if weight.device.type != "cuda":
        inner, scales_zeros = inner.to(weight.device), scales_zeros.to(weight.device)
    return inner.contiguous(), scales_zeros.contiguous()


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
        out = gemv_traceable(
            flat.to(torch.bfloat16),
            self.weight_int4,
            W_INT4_ZP,
            self.out_features,
            sc0=self.scales_zeros,
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
