"""Shared helpers for the tests (not collected: no test_ prefix)."""

from __future__ import annotations

import numpy as np
import torch

from oracle import bz_oracle as O


def bf16_tensor(bits: np.ndarray, device="cuda") -> torch.Tensor:
    """uint16 bf16 bit patterns -> torch.bfloat16 tensor."""
    t = torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16))
    return t.view(torch.bfloat16).to(device)


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def u8_tensor(a: np.ndarray, device="cuda") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).to(device)


class Int4Case:
    """Oracle-quantized int4 weight, uploaded in the GPU path's layout."""

    def __init__(self, w: np.ndarray, group: int = 128, symmetric: bool = False, device="cuda"):
        self.N, self.K = w.shape
        self.group = group
        if symmetric:
            self.q, self.s, self.z = O.quantize_int4_sym(w, group)
            self.lo = -8.0 * self.s
        else:
            self.q, self.s, self.lo, self.z = O.quantize_int4_asym(w, group)
        self.packed = O.pack_nibbles_even_low(self.q)
        self.sz_bits = O.scales_zeros(self.s, self.z)              # [G, N, 2]
        self.s_bits = O.f32_to_bf16_bits(self.s)                    # [N, G]
        self.m_bits = O.f32_to_bf16_bits(self.lo.astype(np.float32))  # [N, G]
        self.w_zp = O.dequant_int4_zp(self.q, self.sz_bits, group)
        self.w_min = O.dequant_int4_min(self.q, self.s_bits, self.m_bits, group)
        self.d_packed = u8_tensor(self.packed, device)
        self.d_sz = bf16_tensor(self.sz_bits, device)
        self.d_s = bf16_tensor(self.s_bits, device)
        self.d_m = bf16_tensor(self.m_bits, device)


class Fp8Case:
    def __init__(self, w: np.ndarray, floor: float = 1e-12, device="cuda"):
        self.N, self.K = w.shape
        self.codes, self.scale = O._fp8_quant(w, floor)
        self.w_eff = O.dequant_fp8(self.codes, self.scale)
        self.d_codes = u8_tensor(self.codes, device)
        self.d_scale = torch.from_numpy(self.scale.copy()).to(device)
