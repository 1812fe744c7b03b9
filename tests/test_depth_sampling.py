"""The depth graph's sampling filter (breeze_amd.fused.depth_graph.
sampling_probs) against the reference's formulation
(models/cudagraph/depth_decoder_graph.py:510-541): temperature, top-k over a
fixed workspace scattered into a -inf row, then a full sort of that row for
top-p, softmax (CPU)."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from breeze_amd.fused.depth_graph import sampling_probs


def _reference_probs(cfg, temperature, top_k, top_p, max_k):
    """The reference's steps, restated: the second top-p pass sorts the whole
    scattered row."""
    scaled = cfg / temperature
    ranks = torch.arange(max_k)
    k = torch.where(top_k > 0, top_k, torch.full_like(top_k, max_k))
    vals, idx = torch.topk(scaled, max_k)
    vals = torch.where(ranks < k, vals, torch.full_like(vals, float("-inf")))
    scaled = torch.full_like(scaled, float("-inf")).scatter_(1, idx, vals)
    s_logits, s_idx = torch.sort(scaled, descending=True)
    remove = torch.cumsum(F.softmax(s_logits, dim=-1), dim=-1) > top_p
    remove = F.pad(remove[..., :-1], (1, 0), value=False)
    s_logits = torch.where(remove, torch.full_like(s_logits, float("-inf")), s_logits)
    scaled = torch.full_like(scaled, float("-inf")).scatter_(1, s_idx, s_logits)
    return F.softmax(scaled, dim=-1)


@pytest.mark.parametrize("vocab,max_k", [(2051, 1024), (64, 64), (300, 256)])
def test_filter_matches_the_full_sort(vocab, max_k):
    g = torch.Generator().manual_seed(vocab)
    rows = 6
    for trial in range(20):
        cfg = torch.randn(rows, vocab, generator=g) * (1 + 3 * torch.rand(rows, 1, generator=g))
        cfg[:, vocab - 3:] = float("-inf")  # masked codec tokens
        temperature = 0.3 + 1.5 * torch.rand(rows, 1, generator=g)
        top_k = torch.randint(0, max_k + 1, (rows, 1), generator=g)
        top_k[0, 0] = 0
        top_p = torch.rand(rows, 1, generator=g)
        top_p[1, 0] = 1.0
        top_p[2, 0] = 0.0
        ranks = torch.arange(max_k)
        got = sampling_probs(cfg, temperature, top_k, top_p, ranks)
        want = _reference_probs(cfg, temperature, top_k, top_p, max_k)
        assert torch.equal(got > 0, want > 0), trial
        torch.testing.assert_close(got, want, rtol=1e-6, atol=1e-7)


def test_filter_edge_cases():
    cfg = torch.tensor([[0.0, 3.0, 1.0, 2.0, -1.0]])
    one = torch.ones(1, 1)
    ranks = torch.arange(5)
    # top-k 2 keeps indices 1 and 3
    p = sampling_probs(cfg, one, torch.tensor([[2]]), one, ranks)
    assert (p > 0).nonzero()[:, 1].tolist() == [1, 3]
    # top-p 0 keeps only the argmax; top-k 0 means every candidate
    p = sampling_probs(cfg, one, torch.tensor([[0]]), torch.zeros(1, 1), ranks)
    assert (p > 0).nonzero()[:, 1].tolist() == [1]
    p = sampling_probs(cfg, one, torch.tensor([[0]]), one, ranks)
    assert bool((p > 0).all()) and abs(float(p.sum()) - 1) < 1e-6
    # a workspace smaller than the vocabulary keeps only its width
    p = sampling_probs(cfg, one, torch.tensor([[0]]), one, torch.arange(3))
    assert (p > 0).nonzero()[:, 1].tolist() == [1, 2, 3]
