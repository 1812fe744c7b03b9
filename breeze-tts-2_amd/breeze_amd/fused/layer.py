"""Fused decode-step forward of a decoder layer (batch of rows, one token),
mirroring models/fused/layer.py:32-99.

Wraps a transformers Qwen3DecoderLayer (the backbone) or a layer of the same
shape (the depth decoder).  Any call that is not a decode step of at most 4
tokens against a static KV cache goes to the original layer, so prefill and
eager paths are untouched.  A decode step is five launches of libbzgemv.so
plus the attention step:

    qkv  = rms_gemv(x, wqkv, ln1)                       1 launch
    attn = attention_step(qkv, cos, sin, pos, cache)    2 (3 with split > 1)
    h    = rms_gemv(attn, wo, residual=x)               1
    act  = rms_gemv(h, wgu, ln2, SiLU-gate)             1
    out  = rms_gemv(act, wd, residual=h)                1

Differences from the reference, on purpose:
  * an Int4Linear MLP runs gate|up as ONE fused SiLU-gate GEMV and down as one
    residual GEMV over the Int4Linear buffers as they are (FusedWeight.
    from_int4); the reference keeps tinygemm there and needs rmsnorm, two
    matmuls, silu_mul and an add (models/fused/layer.py:51-53, 92-95);
  * Fp8Linear / Int4Linear attention projections are adopted as well (the
    reference reads q_proj.weight and so needs bf16 projections);
  * with transformers >= 5, whose StaticLayer writes at its own fill counter
    (cumulative_length) and whose models pass no cache_position, the step
    position comes from that counter and the counter is advanced by the
    cache-write kernel, so fused and unfused calls on one cache stay in step.
"""

from __future__ import annotations

import inspect

import torch
from torch import nn

from ..attention import attention_step
from ..gemv import EPI_RESIDUAL, EPI_SILU_GATE
from .kernels import FusedWeight, rms_gemv

__all__ = ["FusedDecoderLayer"]


def _kind(mod) -> str:
    return type(mod).__name__


def _adopt(mods, bits: int, paired: bool = False) -> FusedWeight:
    """One FusedWeight over the modules' outputs stacked along N: the
    quantized buffers of Int4Linear / Fp8Linear (re-tiled where the shape
    allows), otherwise the float weights quantized to ``bits`` (16 = bf16).
    ``paired``: the two modules are gate and up of a SiLU-gate MLP."""
    kinds = {_kind(m) for m in mods}
    if kinds == {"Int4Linear"}:
        return FusedWeight.from_int4(*mods, paired=paired)
    if kinds == {"Fp8Linear"}:
        return FusedWeight.from_fp8(*mods, paired=paired)
    if kinds & {"Int4Linear", "Fp8Linear"}:
        raise TypeError(f"cannot fuse a mix of {sorted(kinds)}")
    return FusedWeight(torch.cat([m.weight for m in mods], 0).detach(), bits, paired=paired)


def _bf16(w):
    return None if w is None else w.detach().to(torch.bfloat16).contiguous()


class FusedDecoderLayer(nn.Module):
    def __init__(self, layer: nn.Module, layer_idx: int, mlp_bits: int | None = None, attn_bits: int = 16):
        super().__init__()
        self.orig = layer
        self.layer_idx = layer_idx
        attn = layer.self_attn
        self.eps = float(layer.input_layernorm.variance_epsilon)
        self.hkv = int(attn.config.num_key_value_heads)
        self.hd = int(attn.head_dim)
        self.ln1 = _bf16(layer.input_layernorm.weight)
        self.ln2 = _bf16(layer.post_attention_layernorm.weight)
        qn, kn = getattr(attn, "q_norm", None), getattr(attn, "k_norm", None)
        self.qn = _bf16(qn.weight) if qn is not None else None
        self.kn = _bf16(kn.weight) if kn is not None else None
        self.wqkv = _adopt([attn.q_proj, attn.k_proj, attn.v_proj], attn_bits)
        self.wo = _adopt([attn.o_proj], attn_bits)
        mlp = layer.mlp
        bits = mlp_bits or 16
        self.wgu = _adopt([mlp.gate_proj, mlp.up_proj], bits, paired=True)
        self.wd = _adopt([mlp.down_proj], bits)

    # -- cache helpers (transformers 4.57 and >= 5 StaticLayer) ---------------

    def _layer_cache(self, past_key_values, x):
        layer_cache = past_key_values.layers[self.layer_idx]
        if not getattr(layer_cache, "is_initialized", True):
            z = x.new_zeros(x.shape[0], self.hkv, 1, self.hd)
            n = len(inspect.signature(layer_cache.lazy_initialization).parameters)
            layer_cache.lazy_initialization(*([z, z] if n >= 2 else [z]))
        return layer_cache

    @staticmethod
    def _counter(layer_cache, device):
        c = getattr(layer_cache, "cumulative_length", None)
        if isinstance(c, torch.Tensor) and c.device == device and c.dtype == torch.int64 and c.numel() == 1:
            return c
        return None

    # -- set-up before capture -------------------------------------------------

    def prepare(self, rows: int, cache_len: int) -> None:
        """Run the four decode GEMVs once on ``rows`` zero rows (the library
        accepts every weight at this batch; any GEMV workspace is sized on
        the current stream) and allocate the split-attention workspace of a
        ``cache_len``-position cache, so a decode step can be captured
        without a first-use allocation of either."""
        from .. import attention as _attn

        dev = self.ln1.device
        x = torch.zeros(rows, self.wqkv.K, device=dev, dtype=torch.bfloat16)
        rms_gemv(x, self.wqkv, self.ln1, self.eps)
        a = torch.zeros(rows, self.wo.K, device=dev, dtype=torch.bfloat16)
        h = rms_gemv(a, self.wo, None, epilogue=EPI_RESIDUAL, residual=x)
        act = rms_gemv(h, self.wgu, self.ln2, self.eps, epilogue=EPI_SILU_GATE)
        rms_gemv(act, self.wd, None, epilogue=EPI_RESIDUAL, residual=h)
        hq = (self.wqkv.N - 2 * self.hkv * self.hd) // self.hd
        split = _attn.default_split(cache_len)
        if split > 1:
            _attn._attn_workspace(rows, hq, self.hkv, self.hd, split, dev, torch.cuda.current_stream(dev).cuda_stream)

    # -- forward -----------------------------------------------------------------

    def _tokens_in_turn(self, hidden_states, attention_mask, position_ids, past_key_values, use_cache,
                        cache_position, position_embeddings):
        """T <= 4 new tokens (the depth decoder's two-position start) as T
        single-token steps in order: token t attends to the cache through
        position t, which is what row t of the causal mask allows, so the
        steps reproduce the original layer's T-token call."""
        cos, sin = position_embeddings

        def pick(t, tensor, dim):
            return None if tensor is None else tensor.narrow(dim, t, 1)

        steps = [self.forward(hidden_states.narrow(1, t, 1), attention_mask=attention_mask.narrow(2, t, 1),
                              position_ids=pick(t, position_ids, 1), past_key_values=past_key_values,
                              use_cache=use_cache, cache_position=pick(t, cache_position, 0),
                              position_embeddings=(cos.narrow(1, t, 1), sin.narrow(1, t, 1)))
                 for t in range(hidden_states.shape[1])]
        return torch.cat(steps, dim=1)

    def forward(self, hidden_states, attention_mask=None, position_ids=None, past_key_values=None,
                use_cache=False, cache_position=None, position_embeddings=None, **kwargs):
        layers = getattr(past_key_values, "layers", None)
        T = hidden_states.shape[1]
        if layers is None or position_embeddings is None or attention_mask is None or T > 4:
            if cache_position is not None:
                kwargs["cache_position"] = cache_position
            return self.orig(hidden_states, attention_mask=attention_mask, position_ids=position_ids,
                             past_key_values=past_key_values, use_cache=use_cache,
                             position_embeddings=position_embeddings, **kwargs)
        if T > 1:
            return self._tokens_in_turn(hidden_states, attention_mask, position_ids, past_key_values, use_cache,
                                        cache_position, position_embeddings)
        x = hidden_states[:, 0]
        layer_cache = self._layer_cache(past_key_values, hidden_states)
        counter = self._counter(layer_cache, x.device)
        if cache_position is None:
            if counter is None:
                raise ValueError("decode step without cache_position on a cache with no fill counter")
            cache_position = counter.reshape(1).clone()   # the kernel advances the counter itself
        qkv = rms_gemv(x, self.wqkv, self.ln1, self.eps)
        cos, sin = position_embeddings
        attn = attention_step(qkv, cos, sin, cache_position.reshape(-1)[:1], layer_cache.keys, layer_cache.values,
                              attention_mask, self.qn, self.kn, self.eps, seq_len=counter)
        h = rms_gemv(attn, self.wo, None, epilogue=EPI_RESIDUAL, residual=x)
        act = rms_gemv(h, self.wgu, self.ln2, self.eps, epilogue=EPI_SILU_GATE)
        out = rms_gemv(act, self.wd, None, epilogue=EPI_RESIDUAL, residual=h)
        return out.unsqueeze(1)
