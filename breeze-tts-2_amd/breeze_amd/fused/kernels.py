"""Fused decode kernels (MI355X): the host API of models/fused/kernels.py.

rms_gemv: out = epilogue( rmsnorm(x) @ W^T )  -- ONE launch of a gfx950
GEMV (csrc/bz_gemv.hip), where the reference needs two (rms_gemv_kernel +
gemv_epilogue_kernel, models/fused/kernels.py:201-219).
  W is bf16 (N, K); int4 (N, K/2) packed, even k in the low nibble, with
  per-group scale/min (bits=4, pack_int4); the Int4Linear buffers adopted by
  ``from_int4``; or fp8 e4m3 with a per-row scale.  Quantized weights whose
  shape allows it (N % 16 == 0, int4 K % 128 == 0 with group 128, fp8 K % 64
  == 0) are held in the tiled formats of include/bz_gemv.h, read by the
  streaming kernel; a gate|up weight meant for the SiLU-gate epilogue is
  tiled "paired" so each 16-row block holds 8 gate rows and their 8 up rows.
  epilogue 0: none; 1: silu(gate) * up over a [gate | up] weight, output N/2;
  2: add residual.

Differences from the reference, all on purpose:
  * any number of rows M (the reference asserts M <= 2, :336);
  * no runtime autotune and no global partial buffer (:179-198, :262-286):
    the launch shape comes from a static per-shape rule inside the library;
  * the timing helper replays a graph over weight copies that span >= 1 GiB,
    so MI355X's 256 MB Infinity Cache cannot hold the working set.
"""

from __future__ import annotations

import torch

from ..gemv import (
    EPI_NONE,
    EPI_RESIDUAL,
    EPI_SILU_GATE,
    W_BF16,
    W_FP8,
    W_FP8_TILED,
    W_FP8_TILED_PAIRED,
    W_INT4_MIN,
    W_INT4_TILED,
    W_INT4_TILED_PAIRED,
    W_INT4_ZP,
    gemv_traceable,
    pack_tiled,
    quantize_fp8_device,
    quantize_int4_device,
    tiled_bytes,
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


_TILED_FMT = {
    (8, False): W_FP8_TILED, (8, True): W_FP8_TILED_PAIRED,
    (4, False): W_INT4_TILED, (4, True): W_INT4_TILED_PAIRED,
}


def _tile_rows(bits: int, paired: bool, parts, N: int, K: int):
    """Pack row-major or tiled parts (each (src_wfmt, bytes, scales, rows))
    into one tiled weight of N logical rows, the parts stacked along N in
    order.  Returns None when the shape cannot be tiled."""
    dst = _TILED_FMT[(bits, paired)]
    nbytes = tiled_bytes(dst, N, K)
    if not nbytes:
        return None
    out = None
    row0 = 0
    for src, w, sc, n in parts:
        out = pack_tiled(src, w, K, dst, sc0=sc, n_total=N, row0=row0, out=out)
        row0 += n
    return out


def _stack_shape(mods, paired: bool) -> tuple[int, int]:
    """(N, K) of modules stacked along N; a paired stack is [gate | up]."""
    ks = {m.in_features for m in mods}
    if len(ks) != 1:
        raise ValueError(f"modules with different in_features {sorted(ks)} cannot be stacked")
    if paired and (len(mods) != 2 or mods[0].out_features != mods[1].out_features):
        raise ValueError("a paired weight stacks exactly two modules of equal out_features (gate, up)")
    return sum(m.out_features for m in mods), ks.pop()


class FusedWeight:
    """A weight ready for rms_gemv (models/fused/kernels.py:161-176).  Plain
    attributes bits, N, K, w, s, z; ``group`` and ``layout`` describe the
    bytes of ``w``:
      "bf16"         bits 16, w bf16 (N, K);
      "min"          bits 4, w = q*s + z with z the group min (pack_int4);
      "zp"           bits 4, w = (q-8)*s + z, the Int4Linear scales_zeros,
                     row-major (shapes that cannot be tiled);
      "row"          bits 8, e4m3 (N, K) with the per-row scale s;
      "tiled"        bits 4 or 8, the tiled format, scales inside w (s None);
      "tiled-paired" the same with gate|up rows interleaved per 16-row block
                     for the SiLU-gate epilogue.
    ``paired`` asks for the paired layout: the weight is [gate | up] along N."""

    def __init__(self, weight: torch.Tensor, bits: int = 16, paired: bool = False):
        self.bits = bits
        self.N, self.K = weight.shape
        self.group = GROUP
        self.layout = "min"
        self.s = self.z = None
        if bits == 16:
            w = weight
            if w.device.type != "cuda":
                w = w.to(torch.device("cuda", torch.cuda.current_device()))
            self.w = w.to(torch.bfloat16).contiguous()
            self.layout = "bf16"
        elif bits == 8:
            codes, scale = pack_fp8(weight)
            tiled = _tile_rows(8, paired, [(W_FP8, codes.view(torch.uint8), scale, self.N)], self.N, self.K)
            if tiled is None:
                self.w, self.s, self.layout = codes, scale, "row"
            else:
                self.w, self.layout = tiled, "tiled-paired" if paired else "tiled"
        elif bits == 4:
            self.w, self.s, self.z = pack_int4(weight)
        else:
            raise ValueError(bits)

    @classmethod
    def _assemble(cls, bits: int, group: int, N: int, K: int, layout: str, w, s=None) -> "FusedWeight":
        fw = cls.__new__(cls)
        fw.bits, fw.group, fw.N, fw.K, fw.layout = bits, group, N, K, layout
        fw.w, fw.s, fw.z = w, s, None
        return fw

    @classmethod
    def from_fp8(cls, *mods, paired: bool = False) -> "FusedWeight":
        """Adopt Fp8Linear buffers, stacked along N (models/fused/layer.py:
        20-29): tiled modules re-tiled into one weight (paired for gate|up),
        row-major ones tiled when the stacked shape allows, else
        concatenated as they are."""
        from ..fp8_linear import LAYOUT_TILED as FP8_TILED
        from ..fp8_linear import layout_of as fp8_layout_of
        N, K = _stack_shape(mods, paired)
        if K % 16:
            raise ValueError(f"fp8 weights with in_features {K} (not a multiple of 16) cannot be fused")
        layouts = {fp8_layout_of(m.weight_fp8, m.out_features, m.in_features) for m in mods}
        if layouts == {FP8_TILED}:
            parts = [(W_FP8_TILED, m.weight_fp8.view(torch.uint8), None, m.out_features) for m in mods]
        elif FP8_TILED in layouts:
            raise ValueError("fp8 modules in different layouts cannot be fused")
        else:
            parts = [(W_FP8, m.weight_fp8.view(torch.uint8), m.weight_scale.reshape(-1).float(), m.out_features)
                     for m in mods]
        tiled = _tile_rows(8, paired, parts, N, K)
        if tiled is not None:
            return cls._assemble(8, GROUP, N, K, "tiled-paired" if paired else "tiled", tiled)
        w = torch.cat([m.weight_fp8 for m in mods], 0).contiguous()
        s = torch.cat([m.weight_scale.reshape(-1) for m in mods], 0).float().contiguous()
        return cls._assemble(8, GROUP, N, K, "row", w, s)

    @classmethod
    def from_int4(cls, *mods, paired: bool = False) -> "FusedWeight":
        """Adopt Int4Linear buffers stacked along N, so an int4 MLP runs
        gate|up as one fused SiLU-gate GEMV instead of the reference's
        rmsnorm -> 2 tinygemm -> silu_mul sequence (models/fused/layer.py:
        92-95).  Modules in the tiled layout are re-tiled into one weight
        (paired for gate|up); row-major modules are concatenated."""
        from ..int4_linear import LAYOUT_TILED, layout_of
        groups = {m.group_size for m in mods}
        if len(groups) != 1:
            raise ValueError("int4 modules with different group sizes cannot be fused")
        group = groups.pop()
        N, K = _stack_shape(mods, paired)
        layouts = {layout_of(m.weight_int4, m.out_features, m.in_features) for m in mods}
        if layouts == {LAYOUT_TILED}:
            parts = [(W_INT4_TILED, m.weight_int4.view(torch.uint8), None, m.out_features) for m in mods]
            tiled = _tile_rows(4, paired, parts, N, K)
            if tiled is not None:
                return cls._assemble(4, group, N, K, "tiled-paired" if paired else "tiled", tiled)
        if len(layouts) != 1 or layouts == {LAYOUT_TILED}:
            raise ValueError("int4 modules in different layouts cannot be fused")
        w = torch.cat([m.weight_int4.view(torch.uint8) for m in mods], 0).contiguous()
        s = torch.cat([m.scales_zeros for m in mods], 1).contiguous()
        return cls._assemble(4, group, N, K, "zp", w, s)

    def gemv_args(self) -> dict:
        if self.layout.startswith("tiled"):
            return {"wfmt": _TILED_FMT[(self.bits, self.layout == "tiled-paired")], "w": self.w,
                    "group": self.group}
        if self.bits == 16:
            return {"wfmt": W_BF16, "w": self.w}
        if self.bits == 8:
            return {"wfmt": W_FP8, "w": self.w.view(torch.uint8), "sc0": self.s}
        if self.layout == "zp":
            return {"wfmt": W_INT4_ZP, "w": self.w, "sc0": self.s, "group": self.group}
        return {"wfmt": W_INT4_MIN, "w": self.w, "sc0": self.s, "sc1": self.z, "group": self.group}

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.w, self.s, self.z) if t is not None)

    def clone(self) -> "FusedWeight":
        c = FusedWeight._assemble(self.bits, self.group, self.N, self.K, self.layout, self.w.clone(),
                                  None if self.s is None else self.s.clone())
        c.z = None if self.z is None else self.z.clone()
        return c


def rms_gemv(x, fw: FusedWeight, norm_weight=None, eps: float = 1e-6, epilogue: int = 0, residual=None, out=None):
    """models/fused/kernels.py:334-351, as one launch and for any M.

    The SiLU-gate epilogue of a tiled weight needs the paired layout (each
    row block holds its gate and up rows); over an unpaired tiled [gate | up]
    weight it runs as the GEMV followed by silu_mul: two launches, and gate
    and up rounded to bf16 before the product instead of after it."""
    M, K = x.shape
    assert K == fw.K, "decode GEMV: x width must match the weight"
    N = fw.N
    n_out = N // 2 if epilogue == EPI_SILU_GATE else N
    out_dtype = torch.bfloat16 if residual is None else residual.dtype
    if fw.layout == "tiled-paired" and epilogue != EPI_SILU_GATE:
        raise ValueError("a paired gate|up weight is only read with the SiLU-gate epilogue")
    if fw.layout == "tiled" and epilogue == EPI_SILU_GATE:
        gu = rms_gemv(x, fw, norm_weight, eps)
        y = _silu_mul(gu[:, : N // 2], gu[:, N // 2:])
        if out is not None:
            out.copy_(y)
            return out
        return y
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
    """Average GPU microseconds per call of ``fn``.

    ``fn`` is captured ``iters`` times into one HIP graph on a side stream
    (after one eager call, which sizes any workspace), the graph is replayed
    once to warm up, then ``replays`` times between two events.  Capturing
    many calls in one graph takes the host launch cost out of the figure, as
    a decode step that replays its own graph sees it (the measurement of
    models/fused/kernels.py:222-243)."""
    fn()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side), torch.cuda.graph(graph, stream=side):
        for _ in range(iters):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    graph.replay()
    begin, end = (torch.cuda.Event(enable_timing=True) for _ in range(2))
    begin.record()
    for _ in range(replays):
        graph.replay()
    end.record()
    end.synchronize()
    return 1000.0 * begin.elapsed_time(end) / (iters * replays)


def cold_copies(fw: FusedWeight, budget_bytes: int = 1 << 30, min_copies: int = 2) -> list:
    """Clones of ``fw`` to cycle through in a timing loop: together they span
    at least ``budget_bytes`` (1 GiB by default, four times the Infinity
    Cache), so every call reads its weight from HBM."""
    count = max(min_copies, -(-budget_bytes // max(fw.nbytes(), 1)))
    return [fw.clone() for _ in range(count)]
