"""DepthDecodeGraph (the reference's DepthDecoderGraph loop,
models/cudagraph/depth_decoder_graph.py:487-812) on the GPU.

A small depth decoder is built the way the reference's
BreezeDepthDecoderModel is (models/breeze.py:450-483): a Qwen3 decoder stack
plus an embedding table of num_codebooks * vocab rows, a backbone-hidden
projector, an inputs projector, and a per-codebook head of weight
[C - 1, hidden, vocab] (models/breeze.py:590-612).  The depth layers are the
fused ones (install_fused_depth) and the head is the fp32 HIP head.

* Greedy frames (do_sample = 0): every codebook's combined CFG logits match a
  CPU float32 run of the unfused layers, teacher-forced with the graph's own
  tokens (bar 2e-2, max |diff| / max |ref|: the whole frame runs in bf16 --
  embeddings, projectors, two layers, norm -- against float32, and CFG at 2.5
  scales the row errors by about 1.6; each kernel has its 1e-2 bar in its own
  tests), and each token is the argmax of its logits.
* Replays of the captured graph, with eager work in between, give exactly
  the eager loop's tokens and logits (every replay checked).
* Sampling, with the HIP sampler and with the torch one: top-k keeps the
  sampled token inside the top k of the combined logits, top-p = 0 reduces
  to the argmax, and the sampling distribution is zero outside the kept set;
  the HIP sampler's draws repeat after a reseed.
* A batch smaller than the captured one is padded in the CFG layout; a
  larger one recaptures."""

from __future__ import annotations

import copy
import types

import pytest
import torch
from torch import nn

from breeze_amd.fused.depth_graph import DepthDecodeGraph
from breeze_amd.fused.install import install_fused_depth, static_cache

pytestmark = pytest.mark.gpu

TOL = 1e-2        # two bf16 runs of the same frame (padded vs unpadded batch)
TOL_FRAME = 2e-2  # the bf16 frame against the float32 CPU layers
C, V = 6, 64                  # codebooks, vocab per codebook
HB, AUDIO, HID = 384, 320, 256  # backbone hidden, embedding width, depth hidden


class _CodebooksHead(nn.Module):
    def __init__(self, hidden, num_codebooks, vocab):
        super().__init__()
        self.num_codebooks = num_codebooks
        self.weight = nn.Parameter(torch.empty(num_codebooks - 1, hidden, vocab))


def _depth_decoder(seed=11):
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3Model

    cfg = Qwen3Config(hidden_size=HID, intermediate_size=512, num_attention_heads=4, num_key_value_heads=2,
                      head_dim=64, num_hidden_layers=2, rms_norm_eps=1e-6, max_position_embeddings=64,
                      vocab_size=V)
    cfg._attn_implementation = "eager"
    cfg.num_codebooks = C
    cfg.backbone_hidden_size = HB
    torch.manual_seed(seed)
    m = Qwen3Model(cfg).float().eval()
    m.embed_tokens = nn.Embedding(C * V, AUDIO)
    m.backbone_hidden_state_projector = nn.Linear(HB, AUDIO, bias=False)
    m.inputs_embeds_projector = nn.Linear(AUDIO, HID, bias=False)
    head = _CodebooksHead(HID, C, V)
    with torch.no_grad():
        for p in list(m.parameters()) + [head.weight]:
            if p.dim() == 1:
                p.normal_(1, 0.1)
            else:
                p.normal_(0, 0.5 if p is m.embed_tokens.weight else 0.05)
            p.copy_(p.to(torch.bfloat16).float())
    return cfg, types.SimpleNamespace(model=m, codebooks_head=head)


def _gpu_graph(cfg, dd, B, **kw):
    m = copy.deepcopy(dd.model).to("cuda", torch.bfloat16)
    head = copy.deepcopy(dd.codebooks_head).cuda()
    install_fused_depth(types.SimpleNamespace(depth_decoder=types.SimpleNamespace(model=m)), batch_size=B)
    return DepthDecodeGraph(types.SimpleNamespace(model=m, codebooks_head=head), batch_size=B, debug=True, **kw)


def _cpu_frame_logits(cfg, dd, bh, first, tokens, gs):
    """Combined logits [C - 1, half, V] of the unfused layers in float32 on
    the CPU, fed the given tokens (teacher forcing)."""
    m, w = dd.model, dd.codebooks_head.weight.detach()
    B = bh.shape[0]
    half = B // 2
    S = 2 + (C - 1)
    cache = static_cache(cfg, S, B)
    neg = torch.finfo(torch.float32).min
    s = torch.arange(S)
    out = []

    def layers(h, pos):
        mask = torch.where(s[None, :] <= pos[:, None], 0.0, neg).view(1, 1, len(pos), S).expand(B, 1, len(pos), S)
        pe = m.rotary_emb(h, pos.unsqueeze(0))
        for layer in m.layers:
            h = layer(h, attention_mask=mask, position_ids=pos.unsqueeze(0), past_key_values=cache, use_cache=True,
                      cache_position=pos, position_embeddings=pe)
            h = h[0] if isinstance(h, tuple) else h
        return m.norm(h)

    def combine(lg):
        return lg[half:] + gs * (lg[:half] - lg[half:])

    with torch.no_grad():
        ids = torch.stack([torch.zeros_like(first), first], 1)
        emb = m.embed_tokens(ids)
        emb[:, 0] = m.backbone_hidden_state_projector(bh)
        h = layers(m.inputs_embeds_projector(emb), torch.arange(2))
        out.append(combine(h[:, 1] @ w[0]))
        for i in range(1, C - 1):
            tok = torch.cat([tokens[:, i - 1], tokens[:, i - 1]]) + i * V
            h = layers(m.inputs_embeds_projector(m.embed_tokens(tok.unsqueeze(1))), torch.tensor([i + 1]))
            out.append(combine(h[:, 0] @ w[i]))
    return torch.stack(out)


def _inputs(B, seed):
    g = torch.Generator().manual_seed(seed)
    bh = torch.randn(B, HB, generator=g).to(torch.bfloat16).float()
    first = torch.randint(0, V, (B // 2,), generator=g).repeat(2)
    return bh, first


def _rel(a, b):
    return float((a - b).abs().max() / b.abs().max())


@pytest.mark.parametrize("captured,sampler", [(False, "hip"), (True, "hip"), (True, "torch")])
def test_greedy_frames_match_the_cpu_layers(captured, sampler):
    cfg, dd = _depth_decoder()
    B, gs = 4, 2.5
    g = _gpu_graph(cfg, dd, B, do_sample=False, guidance_scale=gs, sampler=sampler)
    if captured:
        g.capture(num_warmup=1)
    for seed in (1, 2, 3):
        bh, first = _inputs(B, seed)
        toks = g.run(bh.cuda(), first.cuda()).cpu()
        assert toks.shape == (B // 2, C - 1)
        logits = g.debug_logits.cpu()
        assert torch.equal(toks, logits.argmax(-1).T)
        ref = _cpu_frame_logits(cfg, dd, bh, first, toks, gs)
        for i in range(C - 1):
            err = _rel(logits[i], ref[i])
            assert err <= TOL_FRAME, (seed, i, err)


def test_replays_equal_the_eager_loop():
    cfg, dd = _depth_decoder()
    B = 2
    g = _gpu_graph(cfg, dd, B, do_sample=False, guidance_scale=1.7)
    runs = [_inputs(B, s) for s in (5, 6, 7)]
    eager = []
    for bh, first in runs:
        t = g.run(bh.cuda(), first.cuda())
        eager.append((t.cpu(), g.debug_logits.clone().cpu()))
    g.capture(num_warmup=1)
    for rep in range(3):
        for (bh, first), (t_e, l_e) in zip(runs, eager):
            t = g.run(bh.cuda(), first.cuda())
            torch.cuda.synchronize()
            assert torch.equal(t.cpu(), t_e), rep
            assert torch.equal(g.debug_logits.cpu(), l_e), rep
            # eager work between replays
            _ = (torch.randn(1024, device="cuda") * 2).sum().item()


@pytest.mark.parametrize("sampler", ["hip", "torch"])
def test_sampling_respects_top_k_and_top_p(sampler):
    cfg, dd = _depth_decoder()
    B = 4
    g = _gpu_graph(cfg, dd, B, do_sample=True, top_k=3, temperature=1.3, guidance_scale=2.0, sampler=sampler)
    g.capture(num_warmup=1)
    torch.manual_seed(0)
    for seed in range(4):
        bh, first = _inputs(B, 20 + seed)
        toks = g.run(bh.cuda(), first.cuda()).cpu()
        logits, probs = g.debug_logits.cpu(), g.debug_probs.cpu()
        top3 = logits.topk(3, dim=-1).indices  # [C - 1, half, 3]
        for i in range(C - 1):
            for r in range(B // 2):
                assert toks[r, i] in top3[i, r], (seed, i, r)
                kept = probs[i, r] > 0
                assert int(kept.sum()) <= 3 and set(kept.nonzero().flatten().tolist()) <= set(top3[i, r].tolist())
                assert abs(float(probs[i, r].sum()) - 1.0) < 1e-5
    # top_p = 0 keeps only the most likely token: sampling equals greedy
    bh, first = _inputs(B, 40)
    toks = g.run(bh.cuda(), first.cuda(), top_k=0, top_p=0.0).cpu()
    assert torch.equal(toks, g.debug_logits.cpu().argmax(-1).T)
    # per-row parameters: row 0 greedy, row 1 sampled from the top 2
    toks = g.run(bh.cuda(), first.cuda(), do_sample=torch.tensor([0, 1]), top_k=torch.tensor([5, 2]), top_p=1.0).cpu()
    logits = g.debug_logits.cpu()
    assert torch.equal(toks[0], logits[:, 0].argmax(-1))
    top2 = logits[:, 1].topk(2, dim=-1).indices
    assert all(toks[1, i] in top2[i] for i in range(C - 1))
    if sampler == "hip":
        # a reseed repeats the frame's draws exactly; without one they move on
        bh, first = _inputs(B, 41)
        g.reseed(77)
        a = g.run(bh.cuda(), first.cuda(), do_sample=1, top_k=0, top_p=1.0, temperature=3.0).cpu()
        b = g.run(bh.cuda(), first.cuda()).cpu()
        g.reseed(77)
        c = g.run(bh.cuda(), first.cuda()).cpu()
        assert torch.equal(a, c) and not torch.equal(a, b)


def test_smaller_batch_is_padded_and_larger_recaptures():
    cfg, dd = _depth_decoder()
    bh2, first2 = _inputs(2, 50)
    ref = _gpu_graph(cfg, dd, 2, do_sample=False, guidance_scale=2.0)
    ref.capture(num_warmup=1)
    want = ref.run(bh2.cuda(), first2.cuda()).cpu()
    want_logits = ref.debug_logits.cpu()
    g = _gpu_graph(cfg, dd, 4, do_sample=False, guidance_scale=2.0)
    g.capture(num_warmup=1)
    got = g.run(bh2.cuda(), first2.cuda()).cpu()
    assert got.shape == (1, C - 1)
    # the padded batch runs other GEMM shapes (rounding may differ): the
    # logits agree until the tokens do, and a differing token is a near tie
    got_logits = g.debug_logits.cpu()[:, :1]
    for i in range(C - 1):
        assert _rel(got_logits[i], want_logits[i]) <= TOL, i
        if got[0, i] != want[0, i]:
            top2 = want_logits[i, 0].topk(2).values
            assert float(top2[0] - top2[1]) <= TOL * float(want_logits[i].abs().max()), i
            break
    bh6, first6 = _inputs(6, 51)
    toks = g.run(bh6.cuda(), first6.cuda()).cpu()
    assert g.batch_size == 6 and g.graph is not None and toks.shape == (3, C - 1)
    assert torch.equal(toks, g.debug_logits.cpu().argmax(-1).T)
    with pytest.raises(ValueError):
        g.run(bh6[:3].cuda(), first6[:3].cuda())
