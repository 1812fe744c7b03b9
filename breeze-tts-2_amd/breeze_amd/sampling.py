"""CFG + HF-order token sampling on the GPU (bz_sample_cfg, include/bz_sample.h).

One launch per call replaces the depth decoder's sampling sequence
(models/cudagraph/depth_decoder_graph.py:487-558): CFG combination, the
invalid-codec-token mask (models/logits_process.py:7-25), temperature, top-k
over a fixed workspace, top-p, softmax and one multinomial draw per row, or
the argmax for greedy rows.  The draws come from Philox4x32-10 keyed by a
seed in device memory and a per-row draw counter that each call advances, so
a captured graph draws fresh numbers on every replay and a reseed (seed and
counters rewritten) repeats a stream exactly.  The sampled tokens follow the
reference's distribution, not torch's random sequence.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib

__all__ = ["sample_cfg", "SampleState", "MAX_VOCAB", "MAX_TOP_K"]

MAX_VOCAB = 4096
MAX_TOP_K = 1024


class SampleState:
    """Device seed and per-row draw counters of one sampling site."""

    def __init__(self, rows: int, device, seed: int = 0) -> None:
        self.seed = torch.zeros(1, dtype=torch.int64, device=device)
        self.counters = torch.zeros(rows, dtype=torch.int64, device=device)
        self.reseed(seed)

    def reseed(self, seed: int) -> None:
        """New key, counters back to zero (outside a capture)."""
        v = int(seed) & ((1 << 64) - 1)
        self.seed.fill_(v - (1 << 64) if v >= (1 << 63) else v)  # the key's 64 bits as int64
        self.counters.zero_()


def _dev(name, t, dtype, dev, numel=None):
    if t.device != dev or t.dtype != dtype or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous {dtype} tensor on {dev}")
    if numel is not None and t.numel() != numel:
        raise ValueError(f"{name} has {t.numel()} entries, expected {numel}")


def sample_cfg(logits: torch.Tensor, tokens: torch.Tensor, state: SampleState, *, temperature: torch.Tensor,
               top_k: torch.Tensor, top_p: torch.Tensor, do_sample: torch.Tensor,
               guidance: Optional[torch.Tensor] = None, codec_size: Optional[int] = None, max_k: int = MAX_TOP_K,
               cfg_out: Optional[torch.Tensor] = None, probs_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """logits fp32 [B, V] (B = 1, or 2 half: cond rows then uncond rows) ->
    tokens int64 [B] (each sampled token in its row and its uncond twin).
    Per-row parameters: temperature / top_p fp32, top_k / do_sample int64,
    guidance fp32 (B >= 2), half entries each.  max_k is the top-k workspace
    (top_k <= 0 means all of it), at most min(V, 1024)."""
    if logits.device.type != "cuda":
        raise RuntimeError("sample_cfg runs on the GPU (HIP kernel); there is no CPU fallback")
    dev = logits.device
    if logits.dtype != torch.float32 or logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be fp32 [B, V] with unit column stride")
    B, V = logits.shape
    if B < 1 or (B > 1 and B % 2):
        raise ValueError(f"B must be 1 or even (cond + uncond rows), got {B}")
    if V > MAX_VOCAB:
        raise ValueError(f"vocabulary {V} exceeds {MAX_VOCAB}")
    half = 1 if B == 1 else B // 2
    codec = V if codec_size is None else int(codec_size)
    max_k = min(int(max_k), V)
    if not (1 <= codec <= V and 1 <= max_k <= MAX_TOP_K):
        raise ValueError("need 1 <= codec_size <= V and 1 <= max_k <= 1024")
    _dev("tokens", tokens, torch.int64, dev, B)
    _dev("temperature", temperature, torch.float32, dev, half)
    _dev("top_k", top_k, torch.int64, dev, half)
    _dev("top_p", top_p, torch.float32, dev, half)
    _dev("do_sample", do_sample, torch.int64, dev, half)
    _dev("seed", state.seed, torch.int64, dev, 1)
    _dev("counters", state.counters, torch.int64, dev, half)
    if B >= 2:
        if guidance is None:
            raise ValueError("a CFG batch needs guidance")
        _dev("guidance", guidance, torch.float32, dev, half)
    for n, t in (("cfg_out", cfg_out), ("probs_out", probs_out)):
        if t is not None:
            _dev(n, t, torch.float32, dev, half * V)
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    _lib.check(
        _lib.lib().bz_sample_cfg(logits.data_ptr(), logits.stride(0), B, V, codec, max_k, ptr(guidance),
                                 temperature.data_ptr(), top_k.data_ptr(), top_p.data_ptr(), do_sample.data_ptr(),
                                 state.seed.data_ptr(), state.counters.data_ptr(), tokens.data_ptr(),
                                 ptr(cfg_out), ptr(probs_out), _lib.stream_of(logits)),
        "bz_sample_cfg",
    )
    return tokens
