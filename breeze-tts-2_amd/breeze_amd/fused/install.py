"""Install fused decode layers on a model's backbone and depth decoder
(models/fused/install.py:16-70).

The reference runs one dummy decode step per layer after installing, to tune
and compile its Triton kernels outside any graph capture.  Nothing here
tunes (launch shapes come from a static rule in the library), but the step
is kept: it loads libbzgemv.so, checks every layer's shapes against the
kernels' limits and leaves the caching allocator warm, before a caller
captures anything.
"""

from __future__ import annotations

import torch

from .layer import FusedDecoderLayer

__all__ = ["install_fused_backbone", "install_fused_depth", "static_cache"]


def static_cache(config, max_cache_len: int, batch_size: int):
    """transformers' StaticCache for either constructor generation: 4.57 takes
    batch_size, >= 5 sizes the batch lazily from the first update."""
    from transformers import StaticCache

    try:
        return StaticCache(config=config, max_cache_len=max_cache_len, batch_size=batch_size)
    except TypeError:
        return StaticCache(config=config, max_cache_len=max_cache_len)


def _install(stack, max_seq: int, batch_size: int, mlp_bits, attn_bits) -> int:
    n = 0
    for i, layer in enumerate(stack.layers):
        if isinstance(layer, FusedDecoderLayer):
            continue
        stack.layers[i] = FusedDecoderLayer(layer, i, mlp_bits=mlp_bits, attn_bits=attn_bits)
        n += 1
    p = next(stack.parameters())
    dev, dtype = p.device, p.dtype
    cache = static_cache(stack.config, max_seq, batch_size)
    x = torch.zeros(batch_size, 1, stack.config.hidden_size, device=dev, dtype=dtype)
    mask = torch.zeros(batch_size, 1, 1, max_seq, device=dev, dtype=dtype)
    pos = torch.zeros(1, dtype=torch.long, device=dev)
    pos_ids = torch.zeros(batch_size, 1, dtype=torch.long, device=dev)
    with torch.no_grad():
        cos, sin = stack.rotary_emb(x, pos_ids)
        for layer in stack.layers:
            layer(x, attention_mask=mask, position_ids=pos_ids, past_key_values=cache, use_cache=True,
                  cache_position=pos, position_embeddings=(cos, sin))
    del cache
    torch.cuda.synchronize(dev)
    return n


def install_fused_backbone(model, *, batch_size: int = 2, max_seq_len: int = 1024, mlp_bits: int | None = None,
                           attn_bits: int = 16) -> int:
    """Replace every backbone layer by a FusedDecoderLayer; returns how many
    were replaced (models/fused/install.py:16-41)."""
    return _install(model.backbone_model, max_seq_len, batch_size, mlp_bits, attn_bits)


def install_fused_depth(model, *, batch_size: int = 2, mlp_bits: int | None = None, attn_bits: int = 16) -> int:
    """Same for the depth decoder, whose cache holds 2 + num_codebooks
    positions (models/fused/install.py:44-70)."""
    dm = model.depth_decoder.model
    return _install(dm, 2 + dm.config.num_codebooks, batch_size, mlp_bits, attn_bits)
