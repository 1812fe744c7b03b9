"""torch-facing wrappers of the C ABI (include/bz_gemv.h).

Every function here only checks arguments, allocates outputs with torch and
hands raw device pointers plus torch's current HIP stream to libbzgemv.so.
There is no CPU path: tensors must live on a GPU and the library must be
built, otherwise the call raises.

``gemv`` is also registered as the custom op ``breeze_amd::gemv`` with a
shape-only fake implementation, so modules calling it stay traceable by
``torch.compile(fullgraph=True)`` (the reference compiles depth layers that
way, models/cudagraph/depth_decoder_graph.py:164-192) and capturable in HIP
graphs (no allocation, sync or tuning inside the library call).
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib
from . import tuning as _tuning
from ._lib import (
    DT_BF16,
    DT_F32,
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
)

__all__ = [
    "gemv",
    "tiled_bytes",
    "pack_tiled",
    "TILED_FORMATS",
    "rmsnorm",
    "silu_mul",
    "quantize_int4_device",
    "quantize_fp8_device",
    "dequant",
    "dequant_matmul",
    "EPI_NONE",
    "EPI_SILU_GATE",
    "EPI_RESIDUAL",
    "W_INT4_ZP",
    "W_INT4_MIN",
    "W_FP8",
    "W_BF16",
    "W_INT4_TILED",
    "W_INT4_TILED_PAIRED",
    "W_FP8_TILED",
    "W_FP8_TILED_PAIRED",
]

TILED_FORMATS = (W_INT4_TILED, W_INT4_TILED_PAIRED, W_FP8_TILED, W_FP8_TILED_PAIRED)

_DT = {torch.bfloat16: DT_BF16, torch.float32: DT_F32}


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _require_gpu(name: str, t: torch.Tensor, device: torch.device) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(f"{name} must be a GPU tensor (got {t.device}); the HIP path has no CPU fallback")
    if t.device != device:
        raise RuntimeError(f"{name} is on {t.device}, expected {device}")


def _rows_aligned(x: torch.Tensor) -> torch.Tensor:
    """bf16 [M,K] view whose rows start on 16-byte boundaries (copy if not)."""
    if x.dtype != torch.bfloat16:
        x = x.to(torch.bfloat16)
    if x.stride(1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
        if x.data_ptr() % 16:
            x = x.clone()
    return x


def gemv(
    x: torch.Tensor,
    w: torch.Tensor,
    wfmt: int,
    n: int,
    *,
    sc0: Optional[torch.Tensor] = None,
    sc1: Optional[torch.Tensor] = None,
    group: int = 128,
    gamma: Optional[torch.Tensor] = None,
    eps: float = 1e-6,
    epilogue: int = EPI_NONE,
    residual: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
    out_dtype: torch.dtype = torch.bfloat16,
    cfg: tuple = (0, 0, 0, 0, 0),
    out2: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """out[M, N_out] = epilogue(rmsnorm?(x) @ w_eff^T) in one launch.

    ``out2`` [M, n2] (tiled formats only, out's dtype, n2 <= N_out): columns
    [0, n2) of the result are stored there as well, by the same launch.

    ``cfg`` (depth, waves, tiles, path[, slices]) all zero takes the static
    per-arch table's launch shape for this GEMV if it has one (tuning.py),
    else the library's built-in rule.

    x [M, K] (any float dtype; computed as bf16), weight of format ``wfmt``
    with ``n`` rows, optional RMSNorm gamma [K], epilogue NONE / SILU_GATE
    (N_out = n/2) / RESIDUAL (residual [M, N_out]).  Returns ``out``.
    """
    if x.dim() != 2:
        raise ValueError(f"x must be 2-D [M, K], got {tuple(x.shape)}")
    dev = x.device
    _require_gpu("x", x, dev)
    _require_gpu("w", w, dev)
    M, K = x.shape
    n_out = n // 2 if epilogue == EPI_SILU_GATE else n
    x = _rows_aligned(x)
    if gamma is not None:
        _require_gpu("gamma", gamma, dev)
        gamma = gamma.to(torch.bfloat16).contiguous()
        if gamma.numel() != K:
            raise ValueError(f"gamma has {gamma.numel()} elements, K = {K}")
    res_dt = DT_BF16
    if epilogue == EPI_RESIDUAL:
        if residual is None:
            raise ValueError("residual epilogue needs a residual tensor")
        _require_gpu("residual", residual, dev)
        if residual.dtype not in _DT:
            residual = residual.to(out.dtype if out is not None else out_dtype)
        if residual.shape != (M, n_out):
            raise ValueError(f"residual shape {tuple(residual.shape)} != {(M, n_out)}")
        if residual.stride(1) != 1:
            residual = residual.contiguous()
        res_dt = _DT[residual.dtype]
    if out is None:
        out = torch.empty(M, n_out, device=dev, dtype=out_dtype)
    else:
        _require_gpu("out", out, dev)
        if out.dtype not in _DT or out.shape != (M, n_out) or out.stride(1) != 1:
            raise ValueError("out must be a bf16/fp32 [M, N_out] row-major tensor")
    if out2 is not None:
        _require_gpu("out2", out2, dev)
        if out2.dim() != 2 or out2.dtype != out.dtype or out2.shape[0] != M or out2.stride(1) != 1 \
                or not 0 < out2.shape[1] <= n_out:
            raise ValueError(f"out2 must be a row-major [M, <= {n_out}] tensor of out's dtype")
    for name, t in (("sc0", sc0), ("sc1", sc1)):
        if t is not None:
            _require_gpu(name, t, dev)
    _check_weight(w, wfmt, n, K, group, sc0, sc1)
    if M == 0:  # no rows: the empty result, nothing launched (the library rejects M = 0)
        return out
    d = _lib.GemvDesc()
    d.abi_version = _lib.ABI_VERSION
    d.M, d.N, d.K = M, n, K
    d.group = group
    d.wfmt = wfmt
    d.epilogue = epilogue
    d.out_dtype = _DT[out.dtype]
    d.residual_dtype = res_dt
    cfg = (tuple(cfg) + (0, 0, 0, 0, 0))[:5]
    if cfg == (0, 0, 0, 0, 0):
        found = _tuning.lookup(dev, n, K, wfmt, epilogue, gamma is not None, M)
        # an entry forcing a matrix-core path (2, 3, 4) is tuned for int4
        # group 128 and cannot run a smaller group: the built-in rule decides
        if found and not (wfmt in (W_INT4_ZP, W_INT4_MIN) and group < 128 and found[3] in (2, 3, 4)):
            cfg = (tuple(found) + (0, 0, 0, 0, 0))[:5]
    d.cfg_depth, d.cfg_waves, d.cfg_tiles, d.cfg_path, d.cfg_slices = cfg
    d.eps = eps
    d.x, d.ldx = x.data_ptr(), x.stride(0)
    d.w = w.data_ptr()
    d.sc0 = _ptr(sc0)
    d.sc1 = _ptr(sc1)
    d.gamma = _ptr(gamma)
    if epilogue == EPI_RESIDUAL:
        d.residual, d.ldr = residual.data_ptr(), residual.stride(0)
    d.out, d.ldo = out.data_ptr(), out.stride(0)
    if out2 is not None:
        d.out2, d.ldo2, d.n_out2 = out2.data_ptr(), out2.stride(0), out2.shape[1]
    stream = _lib.stream_of(x)
    if M >= _TILE_MIN_ROWS or cfg[3] in (_PATH_TILE, _PATH_PANEL):
        need = _lib.lib().bz_gemv_workspace(ctypes.byref(d))
        if need:
            ws = _workspace(dev, stream, need)
            d.workspace, d.workspace_bytes = ws.data_ptr(), ws.numel() * 4
    _lib.check(_lib.lib().bz_gemv(ctypes.byref(d), stream), "bz_gemv")
    return out


def _weight_spec(wfmt: int, n: int, k: int, group: int):
    """(bytes of w, (dtype, numel) of sc0 or None, of sc1 or None) a GEMV of
    this format and shape reads; None when the format is unknown."""
    if wfmt == W_INT4_ZP:
        return n * k // 2, (torch.bfloat16, (k // group) * n * 2), None
    if wfmt == W_INT4_MIN:
        g = k // group
        return n * k // 2, (torch.bfloat16, n * g), (torch.bfloat16, n * g)
    if wfmt == W_FP8:
        return n * k, (torch.float32, n), None
    if wfmt == W_BF16:
        return 2 * n * k, None, None
    if wfmt in TILED_FORMATS:
        return tiled_bytes(wfmt, n, k), None, None
    return None


def _check_weight(w, wfmt, n, k, group, sc0, sc1) -> None:
    """The weight and scale buffers must hold exactly what the kernel reads for
    (wfmt, n, k, group): a short, mis-shaped or strided buffer would be read
    past its end on the GPU.  Raises ValueError (the library checks sizes it
    can see; buffer lengths it cannot)."""
    if wfmt in (W_INT4_ZP, W_INT4_MIN) and (group <= 0 or k % group):
        return  # the library reports the shape error
    spec = _weight_spec(wfmt, n, k, group)
    if spec is None:
        return  # unknown format: the library rejects it
    wbytes, s0, s1 = spec
    if not w.is_contiguous():
        raise ValueError("weight buffer must be contiguous")
    if wfmt in TILED_FORMATS and not wbytes:
        raise ValueError(f"a {n}x{k} weight cannot be tiled (rows % 16, K % unit)")
    if w.numel() * w.element_size() != wbytes:
        raise ValueError(f"weight buffer holds {w.numel() * w.element_size()} bytes, format {wfmt} with "
                         f"N={n}, K={k} needs {wbytes}")
    for name, t, want in (("sc0", sc0, s0), ("sc1", sc1, s1)):
        if want is None:
            continue
        if t is None:
            raise ValueError(f"{name} is required for weight format {wfmt}")
        dt, numel = want
        if t.dtype != dt or t.numel() != numel or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous {dt} tensor of {numel} elements for format {wfmt} "
                             f"(N={n}, K={k}, group={group}); got {t.dtype} {tuple(t.shape)}")


def tiled_bytes(wfmt: int, n: int, k: int) -> int:
    """Bytes of a tiled weight (bz_tiled_bytes); 0 when the shape cannot be tiled."""
    return int(_lib.lib().bz_tiled_bytes(wfmt, n, k))


def pack_tiled(src_wfmt: int, w: torch.Tensor, k: int, dst_wfmt: int, *, sc0: Optional[torch.Tensor] = None,
               n_total: Optional[int] = None, row0: int = 0, out: Optional[torch.Tensor] = None,
               group: int = 128) -> torch.Tensor:
    """Tile the rows of ``w`` (row-major BZ_W_INT4_ZP with scales_zeros
    ``sc0``, BZ_W_FP8 with row scales ``sc0``, or an unpaired tiled weight)
    into logical rows [row0, row0 + n) of a ``dst_wfmt`` weight of
    ``n_total`` rows (default n).  ``out`` (uint8, tiled_bytes bytes) is
    allocated zero-filled when omitted.  Returns ``out``."""
    _require_gpu("w", w, w.device)
    if src_wfmt in (W_INT4_ZP, W_FP8):
        row_bytes = k // 2 if src_wfmt == W_INT4_ZP else k
        n = (w.numel() * w.element_size()) // row_bytes
        if sc0 is None:
            raise ValueError("a row-major source needs its scales (sc0)")
        _check_weight(w, src_wfmt, n, k, group, sc0, None)
    elif src_wfmt in (W_INT4_TILED, W_FP8_TILED):
        per16 = tiled_bytes(src_wfmt, 16, k)
        if not per16 or (w.numel() * w.element_size()) % per16:
            raise ValueError("source is not a whole number of tiled row blocks")
        n = 16 * (w.numel() * w.element_size()) // per16
    else:
        raise ValueError(f"cannot tile from weight format {src_wfmt}")
    n_total = n if n_total is None else n_total
    nbytes = tiled_bytes(dst_wfmt, n_total, k)
    if not nbytes:
        raise ValueError(f"a {n_total}x{k} weight cannot be tiled as format {dst_wfmt}")
    if out is None:
        out = torch.zeros(nbytes, device=w.device, dtype=torch.uint8)
    elif out.numel() * out.element_size() != nbytes or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous buffer of {nbytes} bytes")
    _lib.check(
        _lib.lib().bz_pack_tiled(src_wfmt, w.data_ptr(), _ptr(sc0), n, k, group, dst_wfmt, out.data_ptr(), n_total,
                                 row0, _lib.stream_of(w)),
        "bz_pack_tiled",
    )
    return out


# The several-row kernels (tile, path 4; panel, path 6) run from this many
# rows on; with more than one K slice they need a workspace (fp32 split-K
# partials and arrival counters) that is zero-filled once and left zeroed by
# every call.
_TILE_MIN_ROWS = 5
_PATH_TILE = 4
_PATH_PANEL = 6
_GEMV_WS: dict = {}          # (device index, raw stream, capture id or None) -> int32 buffer
_GEMV_WS_RETIRED: list = []  # outgrown workspaces: a captured graph may still point at one


def _workspace(dev: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    """The GEMV workspace of (device, stream), grown to at least nbytes.

    Each stream has its own, and so has each graph capture (allocated from
    the graph's pool with its zero fill recorded into the graph), so tile-path
    GEMVs on different streams, or in graphs replayed on different streams,
    never share one; the reference keeps one cached split-K buffer per device
    for every stream (models/fused/kernels.py:179,192-198).  Calls on one
    stream run in order and may share it."""
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    return _lib.stream_workspace(_GEMV_WS, (key,), nbytes, torch.device("cuda", key), stream, _GEMV_WS_RETIRED)


# ---- custom-op registration (torch.compile / fake tensors) -----------------


@torch.library.custom_op("breeze_amd::gemv", mutates_args=())
def gemv_op(
    x: torch.Tensor,
    w: torch.Tensor,
    sc0: Optional[torch.Tensor],
    sc1: Optional[torch.Tensor],
    gamma: Optional[torch.Tensor],
    residual: Optional[torch.Tensor],
    wfmt: int,
    n: int,
    group: int,
    eps: float,
    epilogue: int,
    out_f32: bool,
) -> torch.Tensor:
    return gemv(
        x, w, wfmt, n, sc0=sc0, sc1=sc1, group=group, gamma=gamma, eps=eps, epilogue=epilogue,
        residual=residual, out_dtype=torch.float32 if out_f32 else torch.bfloat16,
    )


@gemv_op.register_fake
def _gemv_fake(x, w, sc0, sc1, gamma, residual, wfmt, n, group, eps, epilogue, out_f32):
    n_out = n // 2 if epilogue == EPI_SILU_GATE else n
    return x.new_empty((x.shape[0], n_out), dtype=torch.float32 if out_f32 else torch.bfloat16)


def gemv_traceable(x, w, wfmt, n, *, sc0=None, sc1=None, group=128, gamma=None, eps=1e-6,
                   epilogue=EPI_NONE, residual=None, out_dtype=torch.bfloat16):
    """``gemv`` through the registered custom op while torch.compile traces,
    the direct (cheaper) ctypes call otherwise."""
    if torch.compiler.is_compiling():
        return torch.ops.breeze_amd.gemv(
            x, w, sc0, sc1, gamma, residual, wfmt, n, group, eps, epilogue, out_dtype == torch.float32
        )
    return gemv(x, w, wfmt, n, sc0=sc0, sc1=sc1, group=group, gamma=gamma, eps=eps,
                epilogue=epilogue, residual=residual, out_dtype=out_dtype)


def stream_read(buf: Optional[torch.Tensor], sink: torch.Tensor, chunk: int = 16384, key: int = 0x9E3779B9) -> None:
    """Launch the read-floor kernel over ``buf`` (one workgroup per ``chunk``
    contiguous bytes; the bytes a multiple of it; None: one empty
    workgroup).  ``sink`` is an int32 device tensor, written only if a
    thread's XOR of its data equals ``key``."""
    _require_gpu("sink", sink, sink.device)
    nbytes = 0 if buf is None else buf.numel() * buf.element_size()
    if buf is not None and not buf.is_contiguous():
        raise ValueError("buf must be contiguous")
    _lib.check(_lib.lib().bz_stream_read(_ptr(buf), nbytes, chunk, key, sink.data_ptr(), _lib.stream_of(sink)),
               "bz_stream_read")


def shared_read(x: torch.Tensor, w: Optional[torch.Tensor], wchunk: int, workgroups: int, sink: torch.Tensor,
                key: int = 0x9E3779B9) -> None:
    """Launch the whole-K read floor: ``workgroups`` workgroups each read all
    of ``x`` and their own ``wchunk`` bytes of ``w`` (workgroup b at byte
    b * wchunk; ``w`` must hold workgroups * wchunk bytes).  ``sink`` as for
    stream_read."""
    _require_gpu("sink", sink, sink.device)
    for name, t in (("x", x), ("w", w)):
        if t is not None and not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    wbytes = 0 if w is None else w.numel() * w.element_size()
    if wbytes < workgroups * wchunk:
        raise ValueError(f"w holds {wbytes} bytes, {workgroups} x {wchunk} needed")
    _lib.check(_lib.lib().bz_shared_read(x.data_ptr(), x.numel() * x.element_size(), _ptr(w), wchunk, workgroups,
                                         key, sink.data_ptr(), _lib.stream_of(sink)), "bz_shared_read")


# ---- glue kernels ------------------------------------------------------------


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-6, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """bf16(x * rsqrt(mean(x^2)+eps) * w) per row (models/fused/kernels.py:552-557)."""
    _require_gpu("x", x, x.device)
    x = x.to(torch.bfloat16)
    if x.stride(1) != 1:
        x = x.contiguous()
    M, K = x.shape
    w = w.to(torch.bfloat16).contiguous()
    if out is None:
        out = torch.empty(M, K, device=x.device, dtype=torch.bfloat16)
    _lib.check(
        _lib.lib().bz_rmsnorm(x.data_ptr(), x.stride(0), w.data_ptr(), eps, out.data_ptr(), out.stride(0), M, K,
                              _lib.stream_of(x)),
        "bz_rmsnorm",
    )
    return out


def silu_mul(g: torch.Tensor, u: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """silu(g) * u, bf16 (models/fused/kernels.py:570-575)."""
    _require_gpu("g", g, g.device)
    g = g.to(torch.bfloat16)
    u = u.to(torch.bfloat16)
    if g.stride(1) != 1:
        g = g.contiguous()
    if u.stride(1) != 1:
        u = u.contiguous()
    M, N = g.shape
    if out is None:
        out = torch.empty(M, N, device=g.device, dtype=torch.bfloat16)
    _lib.check(
        _lib.lib().bz_silu_mul(g.data_ptr(), g.stride(0), u.data_ptr(), u.stride(0), out.data_ptr(), out.stride(0),
                               M, N, _lib.stream_of(g)),
        "bz_silu_mul",
    )
    return out


# ---- load-time quantizers ----------------------------------------------------


def _weight_on_gpu(weight: torch.Tensor) -> torch.Tensor:
    if weight.device.type != "cuda":
        if not torch.cuda.is_available():
            raise RuntimeError("quantization runs on the GPU (HIP kernel); no GPU is visible")
        weight = weight.to(torch.device("cuda", torch.cuda.current_device()))
    if weight.dtype not in (torch.float32, torch.bfloat16):
        weight = weight.float()
    return weight.contiguous()


def quantize_int4_device(weight: torch.Tensor, group: int, symmetric: bool = False, layout: int = W_INT4_ZP):
    """HIP group quantizer.  Returns (packed uint8 [N, K/2], sc0, sc1) on the
    GPU: layout W_INT4_ZP -> sc0 = scales_zeros bf16 [K/g, N, 2], sc1 None;
    W_INT4_MIN -> sc0 = scale bf16 [N, K/g], sc1 = min bf16 [N, K/g]."""
    w = _weight_on_gpu(weight)
    N, K = w.shape
    if group < 2 or K % group:
        raise ValueError(f"in_features {K} not divisible by group {group}")
    G = K // group
    packed = torch.empty(N, K // 2, device=w.device, dtype=torch.uint8)
    if layout == W_INT4_ZP:
        sc0 = torch.empty(G, N, 2, device=w.device, dtype=torch.bfloat16)
        sc1 = None
    else:
        sc0 = torch.empty(N, G, device=w.device, dtype=torch.bfloat16)
        sc1 = torch.empty(N, G, device=w.device, dtype=torch.bfloat16)
    _lib.check(
        _lib.lib().bz_quantize_int4(w.data_ptr(), _DT[w.dtype], N, K, group, int(symmetric), layout,
                                    packed.data_ptr(), sc0.data_ptr(), _ptr(sc1), _lib.stream_of(w)),
        "bz_quantize_int4",
    )
    return packed, sc0, sc1


def quantize_fp8_device(weight: torch.Tensor, amax_floor: float):
    """HIP per-row fp8 quantizer.  Returns (codes float8_e4m3fn [N,K], scale f32 [N])."""
    w = _weight_on_gpu(weight)
    N, K = w.shape
    codes = torch.empty(N, K, device=w.device, dtype=torch.uint8)
    scale = torch.empty(N, device=w.device, dtype=torch.float32)
    _lib.check(
        _lib.lib().bz_quantize_fp8(w.data_ptr(), _DT[w.dtype], N, K, amax_floor, codes.data_ptr(), scale.data_ptr(),
                                   _lib.stream_of(w)),
        "bz_quantize_fp8",
    )
    return codes.view(torch.float8_e4m3fn), scale


def dequant(wfmt: int, w: torch.Tensor, n: int, k: int, *, sc0=None, sc1=None, group: int = 128) -> torch.Tensor:
    """w_eff float32 [n, k] decoded by the GPU path's own unpacking code."""
    _require_gpu("w", w, w.device)
    _check_weight(w, wfmt, n, k, group, sc0, sc1)
    out = torch.empty(n, k, device=w.device, dtype=torch.float32)
    _lib.check(
        _lib.lib().bz_dequant(wfmt, w.data_ptr(), _ptr(sc0), _ptr(sc1), n, k, group, out.data_ptr(),
                              _lib.stream_of(w)),
        "bz_dequant",
    )
    return out


def dequant_matmul(x: torch.Tensor, w: torch.Tensor, wfmt: int, n: int, k: int,
                   chunk_bytes: int = 16 << 20) -> torch.Tensor:
    """x [M, k] @ w_eff^T -> bf16 [M, n] for prefill-sized M, over an unpaired
    tiled weight (BZ_W_INT4_TILED, group 128, or BZ_W_FP8_TILED).  The weight
    is decoded by the GPU path's own unpacking (bz_dequant) one run of whole
    16-row blocks at a time, at most ``chunk_bytes`` of fp32 per run, each
    run cast to bf16 and multiplied by torch's GEMM into its output columns:
    the transient memory stays bounded whatever the weight's size (a whole
    fp32 copy of a 10240 x 2560 weight would be 105 MB)."""
    if wfmt not in (W_INT4_TILED, W_FP8_TILED):
        raise ValueError(f"dequant_matmul reads the unpaired tiled formats, not format {wfmt}")
    _require_gpu("x", x, x.device)
    _check_weight(w, wfmt, n, k, 128, None, None)
    if x.dim() != 2 or x.shape[1] != k:
        raise ValueError(f"x must be [M, {k}], got {tuple(x.shape)}")
    x = x.to(torch.bfloat16)
    block = tiled_bytes(wfmt, 16, k)
    wb = w.contiguous().view(torch.uint8).reshape(-1)
    rows = max(16, chunk_bytes // (4 * k) // 16 * 16)
    out = torch.empty(x.shape[0], n, device=x.device, dtype=torch.bfloat16)
    for r0 in range(0, n, rows):
        r = min(rows, n - r0)
        part = wb[(r0 // 16) * block:((r0 + r) // 16) * block]
        out[:, r0:r0 + r] = torch.nn.functional.linear(x, dequant(wfmt, part, r, k).to(torch.bfloat16))
    return out
