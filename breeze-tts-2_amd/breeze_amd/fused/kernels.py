"""Fused decode kernels (MI355X): the host API of models/fused/kernels.py.

rms_gemv: out = epilogue( rmsnorm(x) @ W^T )  -- ONE launch of the gfx950
streaming GEMV (csrc/bz_gemv.hip), where the reference needs two
(rms_gemv_kernel + gemv_epilogue_kernel, models/fused/kernels.py:201-219).
  W is bf16 (N, K); int4 (N, K/2) packed, even k in the low nibble, with
  per-group scale/min (bits=4, pack_int4) or the Int4Linear scales_zeros
  (adopted by ``from_int4``); or fp8 e4m3 (N, K) with a per-row scale.
  epilogue 0: none; 1: silu(gate) * up over a [gate | up] weight, output N/2;
  2: add residual.

Differences from the reference, all on purpose:
  * any number of rows M (the reference asserts M <= 2, :336);
  * no runtime autotune and no global partial buffer (:179-198, :262-286):
    the launch shape comes from a static per-shape rule inside the library,
    so a call is capture-safe at any time and reentrant across streams;
  * the cold-copy rotation used for timing spans >= 1 GiB so MI355X's
    256 MB Infinity Cache cannot hold the working set (:246 uses 160 MB).
"""

from __future__ import annotations

import torch

from ..gemv import (
    EPI_NONE,
    EPI_RESIDUAL,
    EPI_SILU_GATE,
    W_BF16,
    W_FP8,
    W_INT4_MIN,
    W_INT4_ZP,
    gemv_traceable,
    quantize_fp8_device,
    quantize_int4_device,
)
from ..attention import attention_step
from ..gemv import rmsnorm as _rmsnorm
from ..gemv import silu_mul as _silu_mul

GROUP = 128

__all__ = [
    "GROUP",
    "FusedWeight",
    "pack_int4",
    "pack_fp8",
    "rms_gemv",
    "attention_step",
    "rmsnorm",
    "silu_mul",
    "graph_time_us",
    "cold_copies",
]


def pack_int4(weight: torch.Tensor, group: int = GROUP):
    """(N, K) float -> packed (N, K/2) uint8, scale (N, K/group) bf16, min
    (N, K/group) bf16.  w ~= q * scale + min, q in 0..15.  Even k in the low
    nibble (models/fused/kernels.py:141-150)."""
    packed, scale, mn = quantize_int4_device(weight, group, False, W_INT4_MIN)
    return packed, scale, mn


def pack_fp8(weight: torch.Tensor):
    """(N, K) float -> fp8 e4m3 (N, K) with a per-row fp32 scale
    (models/fused/kernels.py:153-158, amax floor 1e-8)."""
    return quantize_fp8_device(weight, 1e-8)


class FusedWeight:
    """A weight in one of the three formats, ready for rms_gemv
    (models/fused/kernels.py:161-176).  Plain attributes bits, N, K, w, s, z;
    ``group`` and ``layout`` ("min": w = q*s + z with z the group min;
    "zp": w = (q-8)*s + z, the Int4Linear scales_zeros) describe int4."""

    def __init__(self, weight: torch.Tensor, bits: int = 16):
        self.bits = bits
        self.N, self.K = weight.shape
        self.group = GROUP
        self.layout = "min"
        if bits == 16:
            w = weight
            if w.device.type != "cuda":
                w = w.to(torch.device("cuda", torch.cuda.current_device()))
            self.w = w.to(torch.bfloat16).contiguous()
            self.s = self.z = None
        elif bits == 8:
            self.w, self.s = pack_fp8(weight)
            self.z = None
        elif bits == 4:
            self.w, self.s, self.z = pack_int4(weight)
        else:
            raise ValueError(bits)

    @classmethod
    def from_fp8(cls, *mods) -> "FusedWeight":
        """Adopt Fp8Linear buffers as-is, concatenated along N
        (models/fused/layer.py:20-29)."""
        fw = cls.__new__(cls)
        fw.bits = 8
        fw.group = GROUP
        fw.layout = "row"
        fw.w = torch.cat([m.weight_fp8 for m in mods], 0).contiguous()
        fw.s = torch.cat([m.weight_scale.reshape(-1) for m in mods], 0).float().contiguous()
        fw.z = None
        fw.N, fw.K = fw.w.shape
        return fw

    @classmethod
    def from_int4(cls, *mods) -> "FusedWeight":
        """Adopt Int4Linear buffers (weight_int4 rows, scales_zeros [G, N, 2])
        concatenated along N, so an int4 MLP runs gate|up as one fused
        SiLU-gate GEMV instead of the reference's rmsnorm -> 2 tinygemm ->
        silu_mul sequence (models/fused/layer.py:92-95)."""
        groups = {m.group_size for m in mods}
        if len(groups) != 1:
            raise ValueError("int4 modules with different group sizes cannot be fused")
        fw = cls.__new__(cls)
        fw.bits = 4
        fw.group = groups.pop()
        fw.layout = "zp"
        fw.w = torch.cat([m.weight_int4.view(torch.uint8) for m in mods], 0).contiguous()
        fw.s = torch.cat([m.scales_zeros for m in mods], 1).contiguous()
        fw.z = None
        fw.N = sum(m.out_features for m in mods)
        fw.K = mods[0].in_features
        return fw

    def gemv_args(self) -> dict:
        if self.bits == 16:
            return {"wfmt": W_BF16, "w": self.w}
        if self.bits == 8:
            return {"wfmt": W_FP8, "w": self.w.view(torch.uint8), "sc0": self.s}
        if self.layout == "zp":
            return {"wfmt": W_INT4_ZP, "w": self.w, "sc0": self.s, "group": self.group}
        return {"wfmt": W_INT4_MIN, "w": self.w, "sc0": self.s, "sc1": self.z, "group": self.group}

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.w, self.s, self.z) if t is not None)


def rms_gemv(x, fw: FusedWeight, norm_weight=None, eps: float = 1e-6, epilogue: int = 0, residual=None, out=None):
    """models/fused/kernels.py:334-351, as one launch and for any M."""
    M, K = x.shape
    assert K == fw.K, "decode GEMV: x width must match the weight"
    N = fw.N
    n_out = N // 2 if epilogue == EPI_SILU_GATE else N
    out_dtype = torch.bfloat16 if residual is None else residual.dtype
    args = fw.gemv_args()
    y = gemv_traceable(
        x,
        args.pop("w"),
        args.pop("wfmt"),
        N,
        gamma=norm_weight,
        eps=eps,
        epilogue=epilogue,
        residual=residual if epilogue == EPI_RESIDUAL else None,
        out_dtype=out_dtype if out_dtype in (torch.bfloat16, torch.float32) else torch.bfloat16,
        **args,
    )
    if out is not None:
        out.copy_(y.view(M, n_out))
        return out
    return y


def rmsnorm(x, w, eps=1e-6, out=None):
    return _rmsnorm(x, w, eps, out)


def silu_mul(g, u, out=None):
    return _silu_mul(g, u, out)


def graph_time_us(fn, iters: int = 20, replays: int = 5) -> float:
    """GPU time per call of fn, measured as a HIP graph replay of `iters`
    back-to-back calls (models/fused/kernels.py:222-243)."""
    fn()
    torch.cuda.synchronize()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=st):
            for _ in range(iters):
                fn()
    torch.cuda.current_stream().wait_stream(st)
    g.replay()
    torch.cuda.synchronize()
    s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s_ev.record()
    for _ in range(replays):
        g.replay()
    e_ev.record()
    torch.cuda.synchronize()
    return s_ev.elapsed_time(e_ev) / (replays * iters) * 1000


def cold_copies(fw: FusedWeight, budget_bytes: int = 1 << 30, min_copies: int = 2) -> list:
    """Copies of fw to rotate through so a timing loop streams from HBM: the
    rotation spans >= budget_bytes (default 1 GiB, 4x the Infinity Cache)."""
    nbytes = max(fw.nbytes(), 1)
    n = max(min_copies, -(-budget_bytes // nbytes))
    copies = []
    for _ in range(n):
        c = FusedWeight.__new__(FusedWeight)
        c.bits, c.N, c.K, c.group, c.layout = fw.bits, fw.N, fw.K, fw.group, fw.layout
        c.w = fw.w.clone()
        c.s = fw.s.clone() if fw.s is not None else None
        c.z = fw.z.clone() if fw.z is not None else None
        copies.append(c)
    return copies
