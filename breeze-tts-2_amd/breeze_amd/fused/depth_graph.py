"""HIP-graph depth-decoder loop over fused layers (mirrors
models/cudagraph/depth_decoder_graph.py:72-989).

One captured graph generates codebook tokens 1 .. C-1 of a frame for a batch
of rows, from the backbone's last hidden state and the frame's first codebook
token:

    start    positions 0 and 1 = [projected backbone hidden state, embedding
             of the first codebook token] -> depth layers -> norm -> codebook
             head 0 (fp32) -> CFG + sampling -> token of codebook 1
    step i   position i + 1 = embedding of the previous token (offset into its
             codebook's rows of the embedding table) -> depth layers -> norm
             -> codebook head i -> CFG + sampling -> token of codebook i + 1

The depth layers are FusedDecoderLayer (install_fused_depth): their GEMVs and
attention steps run on libbzgemv.so, the two-position start as two causal
decode steps.  The codebook head is Fp32CodebooksHead (bz_head_f32), which
picks the codebook's matrix on the GPU from the cache position.  Bias-free
embedding projectors run as bf16 GEMVs and the final RMSNorm as bz_rmsnorm;
the rotary tables of the frame's fixed positions are computed once; the
embedding lookups are torch ops.

CFG layout (models/cudagraph/depth_decoder_graph.py:487-558): rows [0, half)
are the conditional rows and rows [half, 2 half) the unconditional ones; the
token sampled from the combined logits goes to both halves.  Sampling follows
the HF order on the combined logits: invalid codec tokens masked, temperature,
top-k (a fixed 1024-wide workspace), top-p, softmax, multinomial; rows with
do_sample = 0 take the argmax of the combined logits.  The sampling
parameters live in per-row device buffers, so they change between replays
without a new capture.  Two samplers:

    "hip"    (default) one bz_sample_cfg launch per codebook step; its own
             Philox4x32-10 stream (seed from torch's generator, or `seed`)
    "torch"  the reference's torch ops (top-k, then top-p over top-k's
             sorted output instead of a second full sort) and
             torch.multinomial, i.e. torch's random stream
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import nn
from torch.nn import functional as F

from ..heads import Fp32CodebooksHead
from ..sampling import SampleState, sample_cfg
from .install import static_cache
from .kernels import FusedWeight, rms_gemv, rmsnorm

__all__ = ["DepthDecodeGraph", "sampling_probs"]


def sampling_probs(cfg: torch.Tensor, temperature: torch.Tensor, top_k: torch.Tensor, top_p: torch.Tensor,
                   ranks: torch.Tensor) -> torch.Tensor:
    """Sampling distribution [rows, vocab] of combined logits in the HF order
    (depth_decoder_graph.py:510-541): temperature, top-k over a fixed
    workspace of len(ranks) (top_k 0 = the whole workspace), top-p, softmax.
    Per-row parameters are [rows, 1].  Top-p works on top-k's sorted output:
    every logit that survives top-k is among those values, so this equals
    sorting the whole row again (the reference) without the full-width sort.
    Graph-safe: fixed shapes, no host synchronisation."""
    max_k = ranks.numel()
    scaled = cfg / temperature
    k = torch.where(top_k > 0, top_k, torch.full_like(top_k, max_k))
    top_vals, top_idx = torch.topk(scaled, max_k)
    top_vals = torch.where(ranks < k, top_vals, torch.full_like(top_vals, float("-inf")))
    remove = torch.cumsum(F.softmax(top_vals, dim=-1), dim=-1) > top_p
    remove = F.pad(remove[..., :-1], (1, 0), value=False)  # the token that crosses top_p stays
    top_vals = torch.where(remove, torch.full_like(top_vals, float("-inf")), top_vals)
    scaled = torch.full_like(scaled, float("-inf")).scatter_(1, top_idx, top_vals)
    return F.softmax(scaled, dim=-1)


class _Projector:
    """A bias-free nn.Linear of the depth stack (the embedding projectors)
    as one bf16 GEMV launch instead of a library GEMM: [..., K] -> [..., N]."""

    def __init__(self, lin: nn.Linear) -> None:
        self.fw = FusedWeight(lin.weight.detach().to(torch.bfloat16).contiguous(), 16)

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        y = rms_gemv(x.reshape(-1, x.shape[-1]).to(torch.bfloat16).contiguous(), self.fw)
        return y.reshape(*x.shape[:-1], self.fw.N)


def _gemv_or_module(mod):
    if type(mod) is nn.Linear and mod.bias is None and mod.in_features % 8 == 0:
        return _Projector(mod)
    return mod


def _real_batch(batch_size: int) -> int:
    """Rows that are sampled: half of a CFG batch (cond + uncond), or the one
    row without CFG (depth_decoder_graph.py:237-240)."""
    return batch_size if batch_size <= 1 else batch_size // 2


class DepthDecodeGraph:
    """Captured depth-decoder loop.  ``depth_decoder`` has ``.model`` (the
    depth stack: ``embed_tokens`` over num_codebooks * vocab rows,
    ``inputs_embeds_projector``, optional ``backbone_hidden_state_projector``,
    ``rotary_emb``, ``layers``, ``norm``, ``config``) and ``.codebooks_head``
    (a BreezeCodebooksHead, weight [C - 1, hidden, vocab], or its
    Fp32CodebooksHead drop-in).

    run(backbone_hidden [B, Hb], first_cb_token [B]) -> [B / 2 (or 1),
    C - 1] int64 codebook tokens; B may be smaller than the captured batch
    (rows are padded in the CFG layout) and any larger batch recaptures.
    """

    def __init__(self, depth_decoder: nn.Module, *, batch_size: int = 2, temperature: float = 0.9,
                 top_k: int = 50, top_p: float = 1.0, do_sample: bool = True, guidance_scale: float = 3.0,
                 num_codebooks: Optional[int] = None, codec_codebook_size: Optional[int] = None,
                 debug: bool = False, sampler: str = "hip", seed: Optional[int] = None):
        if sampler not in ("hip", "torch"):
            raise ValueError(f"sampler must be 'hip' or 'torch', got {sampler!r}")
        self.sampler = sampler
        # the HIP sampler's Philox key: from torch's generator unless given,
        # so torch.manual_seed makes a run reproducible
        self._seed = int(seed) if seed is not None else int(torch.randint(0, 2 ** 62, (1,)).item())
        self.depth_model = depth_decoder.model
        head = depth_decoder.codebooks_head
        self.codebooks_head = head if isinstance(head, Fp32CodebooksHead) else Fp32CodebooksHead(head)
        cfg = self.depth_model.config
        self.config = cfg
        p = next(self.depth_model.parameters())
        self.device, self.dtype = p.device, p.dtype
        self.hidden_size = int(cfg.hidden_size)
        self.backbone_hidden_size = int(getattr(cfg, "backbone_hidden_size", cfg.hidden_size))
        self.vocab_size = int(cfg.vocab_size)
        self.codec_codebook_size = int(codec_codebook_size) if codec_codebook_size is not None else self.vocab_size
        if not 0 < self.codec_codebook_size <= self.vocab_size:
            raise ValueError(f"codec_codebook_size must be in [1, {self.vocab_size}], got {self.codec_codebook_size}")
        self.num_codebooks = int(num_codebooks if num_codebooks is not None else cfg.num_codebooks)
        self.num_decode_codebooks = self.num_codebooks - 1
        if self.num_decode_codebooks < 1 or self.num_decode_codebooks > self.codebooks_head.weight_t.shape[0]:
            raise ValueError(f"{self.num_codebooks} codebooks need {self.num_decode_codebooks} head matrices, "
                             f"the head has {self.codebooks_head.weight_t.shape[0]}")
        self.max_seq = 2 + self.num_decode_codebooks
        self.debug = debug
        dev = self.device
        # Fixed top-k workspace (depth_decoder_graph.py:200-206): any top_k in
        # [1, _max_k] is a buffer update, not a recapture.
        self._max_k = min(1024, self.vocab_size)
        self._topk_ranks = torch.arange(self._max_k, device=dev)
        # every position / offset tensor exists before the capture
        self.prefill_cache_pos = torch.arange(2, device=dev)
        self.decode_cache_positions = [torch.tensor([2 + i], device=dev) for i in range(self.num_decode_codebooks - 1)]
        self.head_prefill_pos = torch.tensor([1], device=dev)
        self.codebook_offsets = [torch.tensor([i * self.vocab_size], dtype=torch.long, device=dev)
                                 for i in range(self.num_decode_codebooks)]
        # per-position work that does not change between frames: the
        # embedding projectors as bf16 GEMVs, the final RMSNorm as one
        # bz_rmsnorm launch, and the rotary tables of the frame's fixed
        # positions (the reference recomputes them every step)
        dm = self.depth_model
        self._inputs_proj = _gemv_or_module(dm.inputs_embeds_projector)
        bproj = getattr(dm, "backbone_hidden_state_projector", None)
        self._backbone_proj = None if bproj is None else _gemv_or_module(bproj)
        nw, neps = getattr(dm.norm, "weight", None), getattr(dm.norm, "variance_epsilon", None)
        self._norm_w = None if nw is None or neps is None else nw.detach().to(torch.bfloat16).contiguous()
        self._norm_eps = None if neps is None else float(neps)
        with torch.no_grad():
            z = torch.zeros(1, 2, self.hidden_size, dtype=self.dtype, device=dev)
            self._pe_start = tuple(t.contiguous() for t in dm.rotary_emb(z, self.prefill_cache_pos.unsqueeze(0)))
            self._pe_decode = [tuple(t.contiguous() for t in dm.rotary_emb(z[:, :1], pos.unsqueeze(0)))
                               for pos in self.decode_cache_positions]
        self._defaults = dict(temperature=float(temperature), top_k=int(top_k), top_p=float(top_p),
                              do_sample=1 if do_sample else 0, guidance_scale=float(guidance_scale))
        if not 0 <= self._defaults["top_k"] <= self._max_k:
            raise ValueError(f"top_k must be in [0, {self._max_k}]")
        self.graph = None
        self._build(batch_size)

    # -- state of one batch size ----------------------------------------------------

    def _build(self, batch_size: int) -> None:
        if batch_size < 1 or (batch_size > 1 and batch_size % 2):
            raise ValueError(f"batch_size must be 1 or even (cond + uncond rows), got {batch_size}")
        dev, dt = self.device, self.dtype
        self.batch_size = batch_size
        self.half = _real_batch(batch_size)
        self.static_cache = static_cache(self.config, self.max_seq, batch_size)
        self.backbone_hidden_buf = torch.zeros(batch_size, self.backbone_hidden_size, dtype=dt, device=dev)
        self.first_cb_token_buf = torch.zeros(batch_size, dtype=torch.long, device=dev)
        self.output_tokens = torch.zeros(batch_size, self.num_decode_codebooks, dtype=torch.long, device=dev)
        self._tok_buf = torch.zeros(batch_size, dtype=torch.long, device=dev)
        self.prefill_input_ids = torch.zeros(batch_size, 2, dtype=torch.long, device=dev)
        d = self._defaults
        self.temperature_buf = torch.full((self.half, 1), d["temperature"], dtype=torch.float32, device=dev)
        self.top_k_buf = torch.full((self.half, 1), d["top_k"], dtype=torch.long, device=dev)
        self.top_p_buf = torch.full((self.half, 1), d["top_p"], dtype=torch.float32, device=dev)
        self.do_sample_buf = torch.full((self.half,), d["do_sample"], dtype=torch.long, device=dev)
        self.guidance_scale = torch.full((self.half, 1), d["guidance_scale"], dtype=torch.float32, device=dev)
        self._sample_state = SampleState(self.half, dev, seed=self._seed) if self.sampler == "hip" else None
        # per-codebook combined logits and sampling distributions (debug)
        self.debug_logits = (torch.zeros(self.num_decode_codebooks, self.half, self.vocab_size,
                                         dtype=torch.float32, device=dev) if self.debug else None)
        self.debug_probs = (torch.zeros(self.num_decode_codebooks, self.half, self.vocab_size,
                                        dtype=torch.float32, device=dev) if self.debug else None)
        # additive causal masks over the max_seq cache slots: the start's two
        # rows and one row per later position
        neg = torch.finfo(dt).min
        s = torch.arange(self.max_seq, device=dev)
        start = torch.where(s[None, :] <= torch.arange(2, device=dev)[:, None], 0.0, neg).to(dt)
        self.prefill_attn = start.view(1, 1, 2, self.max_seq).expand(batch_size, 1, 2, self.max_seq).contiguous()
        self.decode_attn = []
        for pos in range(2, 2 + self.num_decode_codebooks - 1):
            row = torch.where(s <= pos, 0.0, neg).to(dt)
            self.decode_attn.append(row.view(1, 1, 1, self.max_seq).expand(batch_size, 1, 1, self.max_seq).contiguous())
        self.graph = None

    def reset_cache(self) -> None:
        """Zero the cache and its fill counters (outside any capture)."""
        for layer in self.static_cache.layers:
            if getattr(layer, "is_initialized", False):
                layer.keys.zero_()
                layer.values.zero_()
                if isinstance(getattr(layer, "cumulative_length", None), torch.Tensor):
                    layer.cumulative_length.zero_()

    # -- the loop -------------------------------------------------------------------

    def _layers(self, h, mask, cache_pos, pos_emb):
        pos_ids = cache_pos.unsqueeze(0)
        for layer in self.depth_model.layers:
            h = layer(h, attention_mask=mask, position_ids=pos_ids, past_key_values=self.static_cache,
                      use_cache=True, cache_position=cache_pos, position_embeddings=pos_emb)
            h = h[0] if isinstance(h, tuple) else h
        if self._norm_w is None:
            return self.depth_model.norm(h)
        return rmsnorm(h.reshape(-1, h.shape[-1]), self._norm_w, self._norm_eps).reshape(h.shape)

    def reseed(self, seed: int) -> None:
        """New key for the HIP sampler's stream, draw counters back to zero
        (the torch sampler follows torch's generator instead)."""
        self._seed = int(seed)
        if self._sample_state is not None:
            self._sample_state.reseed(self._seed)

    def _cfg_sample(self, logits: torch.Tensor, i: int) -> None:
        """Combined logits of codebook step i -> self._tok_buf (both halves)."""
        if self._sample_state is not None:
            # one launch (bz_sample_cfg): the same filter, its own Philox stream
            sample_cfg(logits[:, 0, :], self._tok_buf, self._sample_state,
                       temperature=self.temperature_buf.view(-1), top_k=self.top_k_buf.view(-1),
                       top_p=self.top_p_buf.view(-1), do_sample=self.do_sample_buf,
                       guidance=self.guidance_scale.view(-1) if self.batch_size >= 2 else None,
                       codec_size=self.codec_codebook_size, max_k=self._max_k,
                       cfg_out=None if self.debug_logits is None else self.debug_logits[i],
                       probs_out=None if self.debug_probs is None else self.debug_probs[i])
            return
        half = self.half
        if self.batch_size >= 2:
            cond, uncond = logits[:half, 0, :], logits[half: 2 * half, 0, :]
            cfg = uncond + self.guidance_scale * (cond - uncond)
        else:
            cfg = logits[:half, 0, :].clone()
        if self.codec_codebook_size < self.vocab_size:
            cfg[:, self.codec_codebook_size: self.vocab_size] = float("-inf")
        if self.debug_logits is not None:
            self.debug_logits[i].copy_(cfg)
        probs = sampling_probs(cfg, self.temperature_buf, self.top_k_buf, self.top_p_buf, self._topk_ranks)
        if self.debug_probs is not None:
            self.debug_probs[i].copy_(probs)
        greedy = torch.argmax(cfg, dim=-1)
        sampled = torch.multinomial(probs, 1).squeeze(-1)
        toks = torch.where(self.do_sample_buf.bool(), sampled, greedy)
        self._tok_buf[:half] = toks
        if self.batch_size >= 2:
            self._tok_buf[half: 2 * half] = toks

    def _full_loop(self) -> None:
        """The whole frame on static buffers (graph-safe: no host sync)."""
        dm = self.depth_model
        self.prefill_input_ids[:, 0] = 0
        self.prefill_input_ids[:, 1] = self.first_cb_token_buf
        emb = dm.embed_tokens(self.prefill_input_ids)  # [B, 2, audio]
        bh = self.backbone_hidden_buf
        if self._backbone_proj is not None:
            bh = self._backbone_proj(bh)
        emb[:, 0] = bh
        h = self._inputs_proj(emb)  # [B, 2, hidden]
        h = self._layers(h, self.prefill_attn, self.prefill_cache_pos, self._pe_start)
        logits = self.codebooks_head(h[:, 1:, :], cache_position=self.head_prefill_pos)  # [B, 1, vocab] fp32
        self._cfg_sample(logits, 0)
        self._tok_buf.clamp_(0, self.vocab_size - 1)
        self.output_tokens[:, 0] = self._tok_buf
        top = self.num_codebooks * self.vocab_size - 1
        for i in range(1, self.num_decode_codebooks):
            tok = (self._tok_buf + self.codebook_offsets[i]).unsqueeze(1).clamp_(0, top)
            h = self._inputs_proj(dm.embed_tokens(tok))  # [B, 1, hidden]
            cache_pos = self.decode_cache_positions[i - 1]
            h = self._layers(h, self.decode_attn[i - 1], cache_pos, self._pe_decode[i - 1])
            logits = self.codebooks_head(h, cache_position=cache_pos)
            self._cfg_sample(logits, i)
            self._tok_buf.clamp_(0, self.vocab_size - 1)
            self.output_tokens[:, i] = self._tok_buf

    # -- capture / run ----------------------------------------------------------------

    @torch.inference_mode()
    def capture(self, num_warmup: int = 3) -> None:
        """Warm up (loads the library, sizes the allocator and the attention
        workspaces) and capture the loop on a side stream
        (depth_decoder_graph.py:775-812)."""
        for _ in range(num_warmup):
            self.reset_cache()
            self._full_loop()
        torch.cuda.synchronize(self.device)
        self.reset_cache()
        self.graph = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(self.graph, stream=s):
                self._full_loop()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize(self.device)

    @torch.inference_mode()
    def replay(self) -> None:
        """Replay the captured frame on the staged inputs (timing loops; the
        cache is not reset: every slot a frame reads it writes first).  The
        capture's RNG state tensors are inference tensors, so replays run
        under inference mode."""
        if self.graph is None:
            raise RuntimeError("capture() first")
        self.graph.replay()

    def ensure_batch_size(self, batch_size: int) -> None:
        """Rebuild the buffers (and recapture when a graph exists) for another
        batch size; sampling parameters keep their defaults."""
        if batch_size == self.batch_size:
            return
        had_graph = self.graph is not None
        self._build(batch_size)
        if had_graph:
            self.capture()

    def _param(self, buf: torch.Tensor, v, n: int, *, name: str = "") -> None:
        """Per-row parameter: a scalar for every row, or n values padded with
        the first (depth_decoder_graph.py:747-768)."""
        if isinstance(v, (bool, int, float)):
            buf.fill_(int(v) if buf.dtype == torch.long else float(v))
            return
        t = torch.as_tensor(v, device=buf.device).reshape(-1).to(buf.dtype)
        if t.numel() != n:
            raise ValueError(f"{name} has {t.numel()} values for {n} rows")
        flat = buf.view(-1)
        flat[:n].copy_(t)
        if n < flat.numel():
            flat[n:].fill_(t[0].item())

    def _rows(self, dst: torch.Tensor, src: torch.Tensor, actual: int) -> None:
        """Copy `actual` rows into the captured batch in the CFG layout
        [cond rows, cond padding, uncond rows, uncond padding]; padding
        repeats the first row of its half."""
        if actual == self.batch_size:
            dst.copy_(src)
            return
        if self.batch_size == 1 or actual == 1:
            dst[:1].copy_(src[:1])
            dst[1:].copy_(src[:1].expand_as(dst[1:]))
            return
        h, bh = actual // 2, self.half
        dst[:h].copy_(src[:h])
        dst[h:bh].copy_(src[:1].expand_as(dst[h:bh]))
        dst[bh: bh + h].copy_(src[h:actual])
        dst[bh + h:].copy_(src[h: h + 1].expand_as(dst[bh + h:]))

    def set_sampling(self, *, temperature=None, top_k=None, top_p=None, do_sample=None, guidance_scale=None,
                     rows: Optional[int] = None) -> None:
        """Update the per-row sampling buffers (scalars or `rows` values)."""
        n = self.half if rows is None else rows
        if top_k is not None:
            kmax = int(top_k) if isinstance(top_k, (int, float)) else int(torch.as_tensor(top_k).max())
            if kmax > self._max_k:
                raise ValueError(f"top_k {kmax} exceeds the {self._max_k}-wide top-k workspace")
            self._param(self.top_k_buf, top_k, n, name="top_k")
        if temperature is not None:
            self._param(self.temperature_buf, temperature, n, name="temperature")
        if top_p is not None:
            self._param(self.top_p_buf, top_p, n, name="top_p")
        if do_sample is not None:
            self._param(self.do_sample_buf, do_sample, n, name="do_sample")
        if guidance_scale is not None:
            self._param(self.guidance_scale, guidance_scale, n, name="guidance_scale")

    @torch.inference_mode()
    def run(self, backbone_hidden: torch.Tensor, first_cb_token: torch.Tensor, *, temperature=None, top_k=None,
            top_p=None, do_sample=None, guidance_scale=None) -> torch.Tensor:
        """One frame: [actual_half, C - 1] int64 tokens (a copy).  A batch
        larger than the captured one rebuilds and recaptures first; without a
        captured graph the loop runs eagerly on the same kernels."""
        actual = backbone_hidden.shape[0]
        if actual != 1 and actual % 2:
            raise ValueError(f"a CFG batch has cond + uncond rows (even), got {actual}")
        if first_cb_token.reshape(-1).shape[0] != actual:
            raise ValueError("first_cb_token needs one token per row")
        if actual > self.batch_size:
            self.ensure_batch_size(actual)
        n = _real_batch(actual)
        self._rows(self.backbone_hidden_buf, backbone_hidden.to(self.dtype), actual)
        self._rows(self.first_cb_token_buf, first_cb_token.reshape(-1).long(), actual)
        self.set_sampling(temperature=temperature, top_k=top_k, top_p=top_p, do_sample=do_sample,
                          guidance_scale=guidance_scale, rows=n)
        self.reset_cache()
        if self.graph is None:
            self._full_loop()
        else:
            self.graph.replay()
        return self.output_tokens[:n].clone()
