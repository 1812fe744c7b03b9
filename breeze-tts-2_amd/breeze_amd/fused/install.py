"""Install fused decode layers on a model's backbone and depth decoder
(models/fused/install.py:16-70: same entry points, keywords and return
value).

After swapping the layers, each one is readied for graph capture by
``FusedDecoderLayer.prepare``: its four decode GEMVs run once on zero rows
of the serving batch, which loads libbzgemv.so (an error if it is missing;
there is no fallback), makes the library accept every weight at that batch
and sizes any GEMV workspace on the current stream; and the split-attention
workspace of the cache length is allocated.  No cache is built and no
attention runs: nothing here tunes (launch shapes come from a static rule in
the library), so no per-shape first call has to happen outside a capture.
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


def _swap_and_prepare(stack, cache_len: int, batch_size: int, mlp_bits, attn_bits) -> int:
    """Wrap every layer of ``stack`` not yet fused; prepare all of them for
    ``batch_size`` rows over a cache of ``cache_len`` positions.  Returns the
    number of layers wrapped by this call."""
    fresh = [i for i, layer in enumerate(stack.layers) if not isinstance(layer, FusedDecoderLayer)]
    for i in fresh:
        stack.layers[i] = FusedDecoderLayer(stack.layers[i], i, mlp_bits=mlp_bits, attn_bits=attn_bits)
    with torch.no_grad():
        for layer in stack.layers:
            layer.prepare(batch_size, cache_len)
    torch.cuda.current_stream().synchronize()
    return len(fresh)


def install_fused_backbone(model, *, batch_size: int = 2, max_seq_len: int = 1024, mlp_bits: int | None = None,
                           attn_bits: int = 16) -> int:
    """Replace every backbone layer by a FusedDecoderLayer; returns how many
    were replaced (models/fused/install.py:16-41)."""
    return _swap_and_prepare(model.backbone_model, max_seq_len, batch_size, mlp_bits, attn_bits)


def install_fused_depth(model, *, batch_size: int = 2, mlp_bits: int | None = None, attn_bits: int = 16) -> int:
    """Same for the depth decoder, whose cache holds 2 + num_codebooks
    positions (models/fused/install.py:44-70)."""
    dm = model.depth_decoder.model
    return _swap_and_prepare(dm, 2 + dm.config.num_codebooks, batch_size, mlp_bits, attn_bits)
