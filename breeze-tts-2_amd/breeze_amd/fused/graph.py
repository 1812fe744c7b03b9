"""HIP-graph decode step over a fused backbone (mirrors the decode step of
models/cudagraph/backbone_graph.py:56-320).

One captured graph runs a whole single-token step for a batch of rows:
rotary embedding of the step's position ids, every decoder layer (the fused
layers of install_fused_backbone: GEMVs and the attention step on
libbzgemv.so), the final norm, the fp32 head (Fp32Linear, heads.py) and the
classifier-free-guidance combination of cond / uncond rows.  All inputs live
in static buffers that the host updates in place before each replay:

    inputs_buf      [B, 1, H]   the step's input embeddings
    cache_position  [1]         KV cache slot (shared by the rows)
    position_ids    [B, 1]      per-row RoPE positions
    attn_mask       [B, 1, 1, S] additive, rebuilt on the device from
                                 pad_lens and the position
                                 (backbone_graph.py:240-252)

The layers are called directly (not through the model's forward), so no
mask construction or shape logic of the model runs inside the capture.
"""

from __future__ import annotations

import torch
from torch import nn

from ..heads import Fp32Linear
from .install import static_cache

__all__ = ["BackboneDecodeGraph"]


class BackboneDecodeGraph:
    def __init__(self, backbone_model: nn.Module, lm_head: nn.Module, *, batch_size: int = 2,
                 max_seq_len: int = 1024, guidance_scale: float = 1.0):
        self.model = backbone_model
        self.lm_head = Fp32Linear(lm_head) if isinstance(lm_head, nn.Linear) else lm_head
        self.batch_size = batch_size
        self.half = batch_size // 2 if batch_size >= 2 else batch_size
        self.max_seq_len = max_seq_len
        self.guidance_scale = float(guidance_scale)
        p = next(backbone_model.parameters())
        dev, dtype = p.device, p.dtype
        self.device = dev
        cfg = backbone_model.config
        self.static_cache = static_cache(cfg, max_seq_len, batch_size)
        self.cache_position = torch.zeros(1, dtype=torch.long, device=dev)
        self.position_ids = torch.zeros(batch_size, 1, dtype=torch.long, device=dev)
        self.pad_lens = torch.zeros(batch_size, dtype=torch.long, device=dev)
        self.kv_indices = torch.arange(max_seq_len, device=dev)
        self.mask_min = torch.finfo(dtype).min
        self.attn_mask = torch.full((batch_size, 1, 1, max_seq_len), self.mask_min, dtype=dtype, device=dev)
        self.inputs_buf = torch.zeros(batch_size, 1, cfg.hidden_size, dtype=dtype, device=dev)
        self.hidden_buf = torch.zeros(batch_size, 1, cfg.hidden_size, dtype=dtype, device=dev)
        vocab = self.lm_head.out_features
        self.logits_buf = torch.zeros(batch_size, vocab, dtype=torch.float32, device=dev)
        self.cfg_logits_buf = torch.zeros(self.half, vocab, dtype=torch.float32, device=dev)
        self.graph = None

    # -- device-side state ---------------------------------------------------------

    def _set_attention_mask(self) -> None:
        """valid[b, s] = pad_lens[b] <= s <= position (in place, no host sync)."""
        kv = self.kv_indices
        valid = (kv >= self.pad_lens.unsqueeze(1)) & (kv <= self.cache_position)
        self.attn_mask.fill_(self.mask_min)
        self.attn_mask[:, 0, 0, :].masked_fill_(valid, 0.0)

    def _decode_step(self) -> None:
        self._set_attention_mask()
        h = self.inputs_buf
        pe = self.model.rotary_emb(h, self.position_ids)
        for layer in self.model.layers:
            h = layer(h, attention_mask=self.attn_mask, position_ids=self.position_ids,
                      past_key_values=self.static_cache, use_cache=True, cache_position=self.cache_position,
                      position_embeddings=pe)
            h = h[0] if isinstance(h, tuple) else h
        h = self.model.norm(h)
        self.hidden_buf.copy_(h)
        self.logits_buf.copy_(self.lm_head(self.hidden_buf[:, -1, :].float()))
        if self.batch_size >= 2:
            cond, uncond = self.logits_buf[: self.half], self.logits_buf[self.half: 2 * self.half]
            self.cfg_logits_buf.copy_(uncond + self.guidance_scale * (cond - uncond))
        else:
            self.cfg_logits_buf.copy_(self.logits_buf[: self.half])

    # -- host API -----------------------------------------------------------------

    def set_step(self, inputs_embeds: torch.Tensor, position: int, position_ids=None) -> None:
        """Stage one step's inputs: embeddings [B, 1, H], cache slot `position`
        and per-row RoPE positions (default: `position` for every row)."""
        self.inputs_buf.copy_(inputs_embeds)
        self.cache_position.fill_(position)
        if position_ids is None:
            self.position_ids.fill_(position)
        else:
            self.position_ids.copy_(torch.as_tensor(position_ids).reshape(self.batch_size, 1))

    @torch.inference_mode()
    def capture(self, num_warmup: int = 2) -> None:
        """Warm up (loads the library, sizes the allocator) and capture one step
        on a side stream, as backbone_graph.py:287-320.  The warm-up writes into
        the cache at the staged position; reset() clears it."""
        for _ in range(num_warmup):
            self._decode_step()
        torch.cuda.synchronize(self.device)
        self.graph = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(self.graph, stream=s):
                self._decode_step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize(self.device)

    @torch.inference_mode()
    def reset(self) -> None:
        for layer in self.static_cache.layers:
            if getattr(layer, "is_initialized", False):
                layer.keys.zero_()
                layer.values.zero_()
                if isinstance(getattr(layer, "cumulative_length", None), torch.Tensor):
                    layer.cumulative_length.zero_()

    @torch.inference_mode()
    def step(self, inputs_embeds: torch.Tensor, position: int, position_ids=None) -> torch.Tensor:
        """One decode step (graph replay once captured); returns the CFG logits
        buffer [B / 2, vocab] fp32 (valid until the next step)."""
        self.set_step(inputs_embeds, position, position_ids)
        if self.graph is None:
            self._decode_step()
        else:
            self.graph.replay()
        return self.cfg_logits_buf
