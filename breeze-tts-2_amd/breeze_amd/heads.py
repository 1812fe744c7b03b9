"""fp32 output heads on the gfx950 head GEMV (bz_head_f32, include/bz_gemv.h).

The reference keeps its two per-frame heads unquantized and runs them in
fp32 "for numerical stability":

* the backbone ``lm_head`` (hidden -> vocab + 1), cast to fp32 and fed the
  last hidden state cast to fp32 (models/cudagraph/backbone_graph.py:69-70,
  273; models/breeze.py:909);
* the depth decoder's ``BreezeCodebooksHead`` (one [hidden][vocab] matrix per
  codebook after the first), whose weight is cast to fp32
  (models/cudagraph/depth_decoder_graph.py:159-161) and whose codebook is
  picked by ``cache_position - 1`` (models/breeze.py:590-612).

``Fp32Linear`` and ``Fp32CodebooksHead`` are drop-ins for those modules.  The
codebook matrix is chosen on the GPU from the cache-position tensor, so a
captured decode step stays free of host synchronisation.  There is no CPU
path: the weights live on the GPU and every call goes to libbzgemv.so.
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import nn

from . import _lib

__all__ = ["head_f32", "Fp32Linear", "Fp32CodebooksHead", "install_fp32_heads"]


def head_f32(x: torch.Tensor, w: torch.Tensor, *, index: Optional[torch.Tensor] = None, index_offset: int = 0,
             out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out[M, N] = x[M, K] @ W^T in fp32.  w is fp32 [N, K] or a stack
    [C, N, K] of which matrix (*index + index_offset) is used (index: device
    int64 scalar, or None for index_offset itself); a selection outside
    [0, C) gives zeros."""
    if x.device.type != "cuda" or w.device.type != "cuda":
        raise RuntimeError("head_f32 runs on the GPU (HIP kernel); the HIP path has no CPU fallback")
    if w.dtype != torch.float32 or not w.is_contiguous():
        raise ValueError("w must be a contiguous float32 tensor")
    stack = w.dim() == 3
    C, N, K = (w.shape if stack else (1, *w.shape))
    x = x.float()
    if x.dim() != 2 or x.shape[1] != K:
        raise ValueError(f"x must be [M, {K}], got {tuple(x.shape)}")
    if x.stride(1) != 1 or x.stride(0) % 4 or x.data_ptr() % 16:
        x = x.contiguous()
    M = x.shape[0]
    if out is None:
        out = torch.empty(M, N, device=x.device, dtype=torch.float32)
    elif out.dtype != torch.float32 or out.shape != (M, N) or out.stride(1) != 1:
        raise ValueError("out must be a float32 [M, N] tensor with unit column stride")
    if index is not None and (index.dtype != torch.int64 or index.device != x.device):
        raise ValueError("index must be an int64 tensor on the GPU")
    _lib.check(
        _lib.lib().bz_head_f32(x.data_ptr(), x.stride(0), M, K, w.data_ptr(), N, N * K, C,
                               None if index is None else index.data_ptr(), index_offset, out.data_ptr(),
                               out.stride(0), _lib.stream_of(x)),
        "bz_head_f32",
    )
    return out


class Fp32Linear(nn.Module):
    """A bias-free Linear evaluated in fp32 (the reference's fp32 lm_head):
    forward(x) = x.float() @ W^T, returned as float32 [..., N]."""

    def __init__(self, linear: nn.Linear) -> None:
        super().__init__()
        if getattr(linear, "bias", None) is not None:
            raise ValueError("Fp32Linear expects a bias-free Linear")
        w = linear.weight.detach()
        if w.device.type != "cuda":
            w = w.to(torch.device("cuda", torch.cuda.current_device()))
        self.in_features = int(w.shape[1])
        self.out_features = int(w.shape[0])
        self.register_buffer("weight", w.float().contiguous())

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shape = x.shape
        y = head_f32(x.reshape(-1, shape[-1]), self.weight)
        return y.reshape(*shape[:-1], self.out_features)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, fp32=True"


class Fp32CodebooksHead(nn.Module):
    """BreezeCodebooksHead in fp32 (models/breeze.py:590-612).

    Holds the weight [C, hidden, vocab] transposed once to [C, vocab, hidden]
    (rows contiguous along hidden for coalesced reads).  forward(hidden_states
    [B, L, hidden], cache_position=None) -> [B, L, vocab] fp32 where position
    i uses codebook i without a cache position and codebook
    cache_position[i] - 1 with one (chosen on the GPU)."""

    def __init__(self, head: nn.Module) -> None:
        super().__init__()
        w = head.weight.detach()
        if w.device.type != "cuda":
            w = w.to(torch.device("cuda", torch.cuda.current_device()))
        self.num_codebooks = int(getattr(head, "num_codebooks", w.shape[0] + 1))
        self.hidden_size = int(w.shape[1])
        self.vocab_size = int(w.shape[2])
        self.register_buffer("weight_t", w.float().transpose(1, 2).contiguous())

    def forward(self, hidden_states: torch.Tensor, cache_position: Optional[torch.Tensor] = None) -> torch.Tensor:
        B, L, H = hidden_states.shape
        if H != self.hidden_size:
            raise ValueError(f"hidden size {H} != {self.hidden_size}")
        x = hidden_states.float()
        out = torch.empty(B, L, self.vocab_size, device=x.device, dtype=torch.float32)
        if cache_position is not None:
            cache_position = cache_position.reshape(-1)
            if cache_position.numel() != L:
                raise ValueError(f"cache_position has {cache_position.numel()} entries for {L} positions")
            if cache_position.dtype != torch.int64:
                cache_position = cache_position.long()
        for i in range(L):
            idx = None if cache_position is None else cache_position[i: i + 1]
            head_f32(x[:, i, :], self.weight_t, index=idx, index_offset=-1 if idx is not None else i,
                     out=out[:, i, :])
        return out

    def extra_repr(self) -> str:
        return f"codebooks={self.weight_t.shape[0]}, hidden={self.hidden_size}, vocab={self.vocab_size}, fp32=True"


def install_fp32_heads(model) -> int:
    """Swap ``model.lm_head`` and ``model.depth_decoder.codebooks_head`` (where
    present) for their fp32 HIP drop-ins; returns how many were replaced."""
    n = 0
    if isinstance(getattr(model, "lm_head", None), nn.Linear):
        model.lm_head = Fp32Linear(model.lm_head)
        n += 1
    depth = getattr(model, "depth_decoder", None)
    head = getattr(depth, "codebooks_head", None)
    if head is not None and not isinstance(head, Fp32CodebooksHead) and getattr(head, "weight", None) is not None \
            and head.weight.dim() == 3:
        depth.codebooks_head = Fp32CodebooksHead(head)
        n += 1
    return n
