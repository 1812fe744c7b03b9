"""torch-facing wrappers of the decode attention C ABI (include/bz_attn.h).

``qkv_rope_cache``, ``attn_decode`` and ``attention_step`` hand raw device
pointers and torch's current HIP stream to libbzgemv.so; nothing here
computes on the CPU and there is no fallback.  ``attention_step``
(models/fused/kernels.py:505-536) is one launch of bz_attn_step; the other two
mirror the reference's separate rope/cache and attention kernels.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from ._lib import DT_BF16, DT_F32, MASK_BOOL

__all__ = ["qkv_rope_cache", "attn_decode", "attention_step", "default_split", "attn_workspace_bytes"]

_DT = {torch.bfloat16: DT_BF16, torch.float32: DT_F32}


def _gpu(name: str, t: torch.Tensor, dev: torch.device) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(f"{name} must be a GPU tensor (got {t.device}); the HIP path has no CPU fallback")
    if t.device != dev:
        raise RuntimeError(f"{name} is on {t.device}, expected {dev}")


def _dtype_code(name: str, t: torch.Tensor) -> int:
    code = _DT.get(t.dtype)
    if code is None:
        raise TypeError(f"{name} must be bfloat16 or float32, got {t.dtype}")
    return code


def _rows(t: torch.Tensor, B: int, name: str) -> tuple[torch.Tensor, int]:
    """(B or 1, ...) -> a [rows, n] view with unit column stride and its row
    stride (0 when one row serves every batch row)."""
    t2 = t.reshape(t.shape[0], -1)
    if t2.stride(1) != 1:
        t2 = t2.contiguous()
    if t2.shape[0] == B:
        return t2, t2.stride(0) if B > 1 else t2.shape[1]
    if t2.shape[0] == 1:
        return t2, 0
    raise ValueError(f"{name} has {t2.shape[0]} rows for a batch of {B}")


def default_split(S: int) -> int:
    return int(_lib.lib().bz_attn_default_split(S))


def attn_workspace_bytes(B: int, HQ: int, HKV: int, D: int, split: int) -> int:
    return int(_lib.lib().bz_attn_workspace(B, HQ, HKV, D, split))


def qkv_rope_cache(qkv, cos, sin, cache_position, keys, values, HQ: int, q_norm_w=None, k_norm_w=None,
                   eps: float = 1e-6, q_buf=None, seq_len: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Per-head q/k RMSNorm + rotate-half RoPE; q -> fp32 [B, HQ, D] (returned),
    new k/v -> keys/values [B, HKV, S, D] at cache_position (kernels.py:376-401).
    seq_len (device int64 scalar, optional) is set to cache_position + 1."""
    dev = qkv.device
    for n, t in (("qkv", qkv), ("cos", cos), ("sin", sin), ("cache_position", cache_position), ("keys", keys),
                 ("values", values)):
        _gpu(n, t, dev)
    B = qkv.shape[0]
    _, HKV, S, D = keys.shape
    if values.shape != keys.shape or values.dtype != keys.dtype:
        raise ValueError("keys and values must have the same shape and dtype")
    if not (keys.is_contiguous() and values.is_contiguous()):
        raise ValueError("the KV cache must be contiguous [B, HKV, S, D]")
    if keys.shape[0] != B:
        raise ValueError(f"cache batch {keys.shape[0]} != qkv batch {B}")
    if qkv.dtype != torch.bfloat16:
        raise TypeError("qkv must be bfloat16")
    if qkv.stride(1) != 1:
        qkv = qkv.contiguous()
    if cache_position.dtype != torch.int64:
        raise TypeError("cache_position must be int64")
    if (q_norm_w is None) != (k_norm_w is None):
        raise ValueError("q_norm_w and k_norm_w come together")
    cos2, ld_cs = _rows(cos, B, "cos")
    sin2, ld_sin = _rows(sin, B, "sin")
    if ld_cs != ld_sin or cos2.dtype != sin2.dtype or cos2.shape[1] != D or sin2.shape[1] != D:
        raise ValueError("cos and sin must share shape, layout and dtype, with D columns")
    if q_buf is None:
        q_buf = torch.empty(B, HQ, D, device=dev, dtype=torch.float32)
    elif q_buf.dtype != torch.float32 or q_buf.shape != (B, HQ, D) or not q_buf.is_contiguous():
        raise ValueError("q_buf must be a contiguous float32 [B, HQ, D] tensor")
    qn = kn = None
    if q_norm_w is not None:
        qn = q_norm_w.to(torch.bfloat16).contiguous()
        kn = k_norm_w.to(torch.bfloat16).contiguous()
    if seq_len is not None:
        _gpu("seq_len", seq_len, dev)
        if seq_len.dtype != torch.int64 or seq_len.numel() != 1:
            raise ValueError("seq_len must be a device int64 scalar")
    _lib.check(
        _lib.lib().bz_qkv_rope_cache(
            qkv.data_ptr(), qkv.stride(0), B, HQ, HKV, D, None if qn is None else qn.data_ptr(),
            None if kn is None else kn.data_ptr(), eps, cos2.data_ptr(), sin2.data_ptr(), _dtype_code("cos", cos2),
            ld_cs, cache_position.data_ptr(), q_buf.data_ptr(), keys.data_ptr(), values.data_ptr(), S,
            _dtype_code("keys", keys), None if seq_len is None else seq_len.data_ptr(), _lib.stream_of(qkv)),
        "bz_qkv_rope_cache",
    )
    return q_buf


_ATTN_WS: dict[tuple, torch.Tensor] = {}
_ATTN_WS_RETIRED: list = []


def _attn_workspace(B, HQ, HKV, D, split, device, stream) -> Optional[torch.Tensor]:
    """Split partials and arrival counters (models/fused/kernels.py:480-489):
    one zeroed buffer per shape, device and stream -- and per graph capture
    while one is under way, with its zero fill recorded into the graph -- so
    split attention steps on different streams, or in graphs replayed on
    different streams, never share one (the reference caches one buffer per
    shape for every stream).  The kernel leaves the counters at zero, so
    calls on one stream reuse the buffer without clearing it."""
    if split <= 1:
        return None
    key = (B, HQ, HKV, D, split, device.index if device.index is not None else torch.cuda.current_device())
    return _lib.stream_workspace(_ATTN_WS, key, attn_workspace_bytes(B, HQ, HKV, D, split), device, stream,
                                 _ATTN_WS_RETIRED)


def _mask_rows(mask: torch.Tensor, B: int, S: int) -> tuple[torch.Tensor, int, int]:
    """(B or 1, 1, 1, >= S) additive or bool mask -> ([rows, >= S] view, dtype
    code, row stride), read in place (models/fused/kernels.py:492-502)."""
    m2 = mask.reshape(mask.shape[0], -1)
    if m2.shape[1] < S:
        raise ValueError(f"mask covers {m2.shape[1]} positions, the cache has {S}")
    if m2.stride(1) != 1:
        m2 = m2.contiguous()
    if mask.dtype == torch.bool:
        m2, code = m2.view(torch.uint8), MASK_BOOL
    else:
        if mask.dtype not in _DT:
            m2 = m2.float()
        code = _DT[m2.dtype]
    if m2.shape[0] == B:
        return m2, code, m2.stride(0) if B > 1 else max(m2.shape[1], S)
    if m2.shape[0] == 1:
        return m2, code, 0
    raise ValueError(f"mask has {m2.shape[0]} rows for a batch of {B}")


def _out_buffer(out, B, HQ, D, dev):
    if out is None:
        return torch.empty(B, HQ * D, device=dev, dtype=torch.bfloat16)
    if out.dtype != torch.bfloat16 or out.shape != (B, HQ * D) or out.stride(1) != 1:
        raise ValueError("out must be a bf16 [B, HQ * D] row-major tensor")
    return out


def attn_decode(q, keys, values, mask, cache_position, out=None, split: Optional[int] = None,
                scale: Optional[float] = None) -> torch.Tensor:
    """softmax(q k^T * scale + mask) v over cache positions [0, pos]; q fp32
    [B, HQ, D] -> bf16 [B, HQ * D] (kernels.py:404-475), one launch."""
    dev = q.device
    for n, t in (("keys", keys), ("values", values), ("mask", mask), ("cache_position", cache_position)):
        _gpu(n, t, dev)
    B, HQ, D = q.shape
    _, HKV, S, _ = keys.shape
    if q.dtype != torch.float32 or not q.is_contiguous():
        raise ValueError("q must be a contiguous float32 [B, HQ, D] tensor")
    m2, mcode, ld_mask = _mask_rows(mask, B, S)
    split = default_split(S) if split is None else split
    ws = _attn_workspace(B, HQ, HKV, D, split, dev, _lib.stream_of(q))
    out = _out_buffer(out, B, HQ, D, dev)
    _lib.check(
        _lib.lib().bz_attn_decode(
            q.data_ptr(), keys.data_ptr(), values.data_ptr(), _dtype_code("keys", keys), B, HQ, HKV, D, S,
            m2.data_ptr(), mcode, ld_mask, cache_position.data_ptr(), D ** -0.5 if scale is None else scale, split,
            None if ws is None else ws.data_ptr(), out.data_ptr(), out.stride(0), _lib.stream_of(q)),
        "bz_attn_decode",
    )
    return out


def attention_step(qkv, cos, sin, cache_position, keys, values, mask, q_norm_w=None, k_norm_w=None, eps=1e-6,
                   out=None, q_buf=None, *, split: Optional[int] = None, seq_len: Optional[torch.Tensor] = None):
    """qkv (B, (HQ + 2 HKV) D) bf16 -> attention output (B, HQ D) bf16, with the
    new k/v written into the static cache (B, HKV, S, D) at cache_position
    (models/fused/kernels.py:505-536).  One launch (bz_attn_step): q/k norm,
    RoPE, the cache write and split attention with its combine.  ``q_buf`` is
    accepted for the reference's signature and unused (q stays on chip)."""
    dev = qkv.device
    for n, t in (("qkv", qkv), ("cos", cos), ("sin", sin), ("cache_position", cache_position), ("keys", keys),
                 ("values", values), ("mask", mask)):
        _gpu(n, t, dev)
    B = qkv.shape[0]
    _, HKV, S, D = keys.shape
    HQ = (qkv.shape[1] - 2 * HKV * D) // D
    if HQ < 1 or (HQ + 2 * HKV) * D != qkv.shape[1]:
        raise ValueError(f"qkv width {qkv.shape[1]} does not split into q/k/v heads of {D} with {HKV} kv heads")
    if values.shape != keys.shape or values.dtype != keys.dtype:
        raise ValueError("keys and values must have the same shape and dtype")
    if not (keys.is_contiguous() and values.is_contiguous()) or keys.shape[0] != B:
        raise ValueError("the KV cache must be contiguous [B, HKV, S, D] with the batch of qkv")
    if qkv.dtype != torch.bfloat16:
        raise TypeError("qkv must be bfloat16")
    if qkv.stride(1) != 1:
        qkv = qkv.contiguous()
    if cache_position.dtype != torch.int64:
        raise TypeError("cache_position must be int64")
    if (q_norm_w is None) != (k_norm_w is None):
        raise ValueError("q_norm_w and k_norm_w come together")
    cos2, ld_cs = _rows(cos, B, "cos")
    sin2, ld_sin = _rows(sin, B, "sin")
    if ld_cs != ld_sin or cos2.dtype != sin2.dtype or cos2.shape[1] != D or sin2.shape[1] != D:
        raise ValueError("cos and sin must share shape, layout and dtype, with D columns")
    qn = kn = None
    if q_norm_w is not None:
        qn = q_norm_w.to(torch.bfloat16).contiguous()
        kn = k_norm_w.to(torch.bfloat16).contiguous()
    if seq_len is not None:
        _gpu("seq_len", seq_len, dev)
        if seq_len.dtype != torch.int64 or seq_len.numel() != 1:
            raise ValueError("seq_len must be a device int64 scalar")
        if seq_len.data_ptr() == cache_position.data_ptr():
            raise ValueError("seq_len must not alias cache_position")
    m2, mcode, ld_mask = _mask_rows(mask, B, S)
    split = default_split(S) if split is None else split
    ws = _attn_workspace(B, HQ, HKV, D, split, dev, _lib.stream_of(qkv))
    out = _out_buffer(out, B, HQ, D, dev)
    _lib.check(
        _lib.lib().bz_attn_step(
            qkv.data_ptr(), qkv.stride(0), B, HQ, HKV, D, None if qn is None else qn.data_ptr(),
            None if kn is None else kn.data_ptr(), eps, cos2.data_ptr(), sin2.data_ptr(), _dtype_code("cos", cos2),
            ld_cs, cache_position.data_ptr(), keys.data_ptr(), values.data_ptr(), S, _dtype_code("keys", keys),
            None if seq_len is None else seq_len.data_ptr(), m2.data_ptr(), mcode, ld_mask, D ** -0.5, split,
            None if ws is None else ws.data_ptr(), out.data_ptr(), out.stride(0), _lib.stream_of(qkv)),
        "bz_attn_step",
    )
    return out
