"""FP8 (OCP e4m3) weight Linear for bandwidth-bound decode, on MI355X.

Drop-in for models/fp8_linear.py: same names (FP8_MAX, FP8_DTYPE,
MIN_QUANT_BYTES, DEFAULT_TARGET_NAMES, Fp8Linear, quantize_module_fp8), same
buffer names and dtypes (``weight_fp8`` float8_e4m3fn, ``weight_scale`` fp32
(1, N)), the codes and scales computed by the same formula
(models/fp8_linear.py:58-66), same stats dict.

``weight_fp8`` holds one of two layouts, told apart by its shape:

  tiled (LAYOUT_TILED, whenever out_features % 16 == 0 and in_features % 64
  == 0 -- every decode shape of the model): [N/16, 16 K + 128], the bytes of
      BZ_W_FP8_TILED (include/bz_gemv.h): per block of 16 output rows, K/64
      tiles of 1 KiB (16 rows x 64 codes) followed by the block's 16 row
      scales, read by the streaming GEMV path (one contiguous chunk per
      workgroup);
  row-major (LAYOUT_ROWMAJOR, any other shape): [N, K], the reference's own
      buffer.

weight_scale stays the reference's (1, N) buffer in both cases (the tiled
layout repeats the scales inside its blocks, 64 bytes per 16 rows).

forward() is the weight-only form: bf16 activations times e4m3 weights with
fp32 accumulation and the per-channel scale applied to the dot product, i.e.
exactly ``x @ (w8.float() * s).T`` of the reference's own correctness
definition (bench_gemv.py:49) and its fused path
(models/fused/kernels.py:84-85,124-126).  The reference's
``Fp8Linear.forward`` additionally rounds the activations to fp8 per row
before ``_scaled_mm`` (models/fp8_linear.py:72-82); that extra rounding is
not reproduced (it only adds error), since decode here is bound by the weight
bytes, not by the arithmetic.  Any in_features is accepted, as in the
reference; rows of a row-major weight whose length is not a multiple of 16
are read from a zero-padded copy.
"""

from __future__ import annotations

import torch
from torch import nn

from ._swap import swap_linears
from .gemv import (W_FP8, W_FP8_TILED, dequant_matmul, gemv_traceable, pack_tiled, quantize_fp8_device,
                   tiled_bytes)

# Max representable magnitude of float8_e4m3fn.
FP8_MAX = 448.0
FP8_DTYPE = torch.float8_e4m3fn

MIN_QUANT_BYTES = 8 * 1024 * 1024

DEFAULT_TARGET_NAMES = ("gate_proj", "up_proj", "down_proj")

# amax floor of Fp8Linear (models/fp8_linear.py:58)
AMAX_FLOOR = 1e-12

# Above this many rows a call is a prefill: a tiled weight is then decoded
# to bf16 in bounded row chunks and multiplied by the library GEMM.
PREFILL_ROWS = 32

# Tags recorded by the checkpoint manifest for the two layouts of weight_fp8
# (the row-major one is the reference's buffer as it is).
LAYOUT_TILED = "bz-fp8-tiled16-v1"
LAYOUT_ROWMAJOR = "e4m3-rowmajor"


def tileable(out_features: int, in_features: int) -> bool:
    """Whether a weight of this shape is stored in the tiled layout."""
    return out_features % 16 == 0 and in_features % 64 == 0


def tiled_shape(out_features: int, in_features: int) -> tuple[int, int]:
    """Shape of a tiled weight_fp8: [N/16, bytes per 16-row block]."""
    return out_features // 16, tiled_bytes(W_FP8_TILED, 16, in_features)


def layout_of(weight_fp8: torch.Tensor, out_features: int, in_features: int) -> str:
    """The layout a weight_fp8 buffer holds, from its shape."""
    if tuple(weight_fp8.shape) == (out_features, in_features):
        return LAYOUT_ROWMAJOR
    return LAYOUT_TILED


def _tile(codes: torch.Tensor, scale: torch.Tensor, out_features: int, in_features: int) -> torch.Tensor:
    """Row-major codes uint8 [N, K] + row scales fp32 [N] -> tiled weight_fp8."""
    t = pack_tiled(W_FP8, codes, in_features, W_FP8_TILED, sc0=scale.reshape(-1).float().contiguous())
    return t.view(FP8_DTYPE).view(*tiled_shape(out_features, in_features))


def retile(module: "Fp8Linear") -> bool:
    """Convert a row-major Fp8Linear (the reference's buffers, e.g. loaded from
    one of its checkpoints) to the tiled layout in place, on its GPU.
    Returns whether it changed."""
    if layout_of(module.weight_fp8, module.out_features, module.in_features) != LAYOUT_ROWMAJOR:
        return False
    if not tileable(module.out_features, module.in_features):
        return False
    module.weight_fp8 = _tile(module.weight_fp8.view(torch.uint8), module.weight_scale, module.out_features,
                              module.in_features)
    return True


class Fp8Linear(nn.Module):
    """Drop-in replacement for a bias-free nn.Linear using FP8 weights."""

    def __init__(self, linear: nn.Linear) -> None:
        super().__init__()
        if linear.bias is not None:
            raise ValueError("Fp8Linear expects a bias-free Linear")

        weight = linear.weight.data
        self.in_features = int(weight.shape[1])
        self.out_features = int(weight.shape[0])

        codes, scale = quantize_fp8_device(weight, AMAX_FLOOR)
        if tileable(self.out_features, self.in_features):
            codes = _tile(codes.view(torch.uint8), scale, self.out_features, self.in_features)
        if weight.device.type != "cuda":
            codes, scale = codes.to(weight.device), scale.to(weight.device)
        self.register_buffer("weight_fp8", codes.contiguous())
        self.register_buffer("weight_scale", scale.reshape(1, -1).contiguous())

    def _gemv_codes(self) -> tuple[torch.Tensor, int]:
        """(row-major codes uint8, row length) as the GEMV reads them.  The GEMV
        streams 16-byte rows; when in_features is not a multiple of 16 the
        rows are padded with zero codes (+0.0) in a copy kept beside the
        reference's buffer and refreshed whenever that buffer changes."""
        codes = self.weight_fp8.view(torch.uint8)
        k = self.in_features
        if k % 16 == 0:
            return codes, k
        k16 = -(-k // 16) * 16
        key = (codes.data_ptr(), codes._version)
        if getattr(self, "_padded_key", None) != key:
            self._padded = torch.nn.functional.pad(codes, (0, k16 - k)).contiguous()
            self._padded_key = key
        return self._padded, k16

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shape = x.shape
        flat = x.reshape(-1, shape[-1]).to(torch.bfloat16)
        N, K = self.out_features, self.in_features
        if layout_of(self.weight_fp8, N, K) == LAYOUT_TILED:
            w = self.weight_fp8.view(torch.uint8)
            if flat.shape[0] > PREFILL_ROWS and not torch.compiler.is_compiling():
                out = dequant_matmul(flat, w, W_FP8_TILED, N, K)
            else:
                out = gemv_traceable(flat, w, W_FP8_TILED, N)
            return out.to(x.dtype).reshape(*shape[:-1], N)
        codes, k = self._gemv_codes()
        if k != K:
            flat = torch.nn.functional.pad(flat, (0, k - K))
        out = gemv_traceable(flat, codes, W_FP8, N, sc0=self.weight_scale)
        return out.to(x.dtype).reshape(*shape[:-1], N)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, fp8=True"


def quantize_module_fp8(
    root: nn.Module,
    *,
    target_names: tuple[str, ...] = DEFAULT_TARGET_NAMES,
    min_bytes: int = MIN_QUANT_BYTES,
) -> dict[str, int]:
    """Swap qualifying Linear layers under ``root`` for FP8 equivalents
    (models/fp8_linear.py:89-122).  Construction errors propagate, as in the
    reference.  Saved bytes: fp8 keeps half of a bf16 weight."""
    st = swap_linears(
        root,
        target_names,
        min_bytes,
        build=Fp8Linear,
        saved_bytes=lambda nbytes: nbytes // 2,
        tolerate_errors=False,
        drop_original=False,
    )
    return {
        "converted": st.converted,
        "skipped_below_threshold": st.small,
        "weight_bytes_saved": st.saved,
    }
