"""bz_sample_cfg (breeze_amd.sampling.sample_cfg) on the GPU: the fused
CFG + HF-order sampler of the depth-decoder loop.

* The combined logits and the sampling distribution it reports match the
  torch formulation (breeze_amd.fused.depth_graph.sampling_probs, itself
  pinned on the CPU to the reference's full-sort steps): same kept set
  (a difference only where the cumulative probability before the boundary
  token is within 1e-5 of top_p) and probabilities within 1e-5.
* Greedy rows return the first argmax; top_k = 1 and top_p = 0 sample the
  argmax.
* Draws follow the distribution: 20480 draws of a 64-token distribution pass
  a chi-square test (fixed seed).
* The stream is reproducible: the same seed and counters give the same
  tokens; every call advances the counters; graph replays advance them too
  and match eager calls made from the same state.
* Each sampled token also lands in its unconditional twin row."""

from __future__ import annotations

import pytest
import torch

from breeze_amd.fused.depth_graph import sampling_probs
from breeze_amd.sampling import SampleState, sample_cfg

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _params(half, temperature=1.0, top_k=0, top_p=1.0, do_sample=1, guidance=2.0):
    f = lambda v, dt: (torch.as_tensor(v, dtype=dt).reshape(-1).expand(half).contiguous().to(DEV))  # noqa: E731
    return dict(temperature=f(temperature, torch.float32), top_k=f(top_k, torch.int64),
                top_p=f(top_p, torch.float32), do_sample=f(do_sample, torch.int64),
                guidance=f(guidance, torch.float32))


def _torch_cfg(logits, half, g, codec):
    cond, uncond = logits[:half], logits[half:]
    cfg = uncond + g.view(-1, 1) * (cond - uncond)
    cfg[:, codec:] = float("-inf")
    return cfg


def test_filter_and_greedy_match_torch():
    gen = torch.Generator(device=DEV).manual_seed(1)
    half, V, codec = 24, 2051, 2048
    logits = torch.randn(2 * half, V, device=DEV, generator=gen) * 3
    prm = _params(half)
    prm["temperature"] = (0.5 + torch.rand(half, device=DEV, generator=gen)).contiguous()
    prm["top_k"] = torch.randint(0, 1025, (half,), device=DEV, generator=gen)
    prm["top_k"][:3] = torch.tensor([0, 1, 1024], device=DEV)
    prm["top_p"] = torch.rand(half, device=DEV, generator=gen).contiguous()
    prm["top_p"][:4] = torch.tensor([1.0, 0.0, 0.9, 1.0], device=DEV)
    prm["guidance"] = (1 + 2 * torch.rand(half, device=DEV, generator=gen)).contiguous()
    prm["do_sample"][half // 2:] = 0  # rows [0, half / 2) sample, the rest are greedy
    tokens = torch.full((2 * half,), -1, dtype=torch.int64, device=DEV)
    cfg_out = torch.empty(half, V, device=DEV)
    probs_out = torch.empty(half, V, device=DEV)
    st = SampleState(half, DEV, seed=7)
    sample_cfg(logits, tokens, st, codec_size=codec, cfg_out=cfg_out, probs_out=probs_out, **prm)
    torch.cuda.synchronize()
    cfg = _torch_cfg(logits, half, prm["guidance"], codec)
    torch.testing.assert_close(cfg_out, cfg, rtol=1e-6, atol=1e-6)
    want = sampling_probs(cfg, prm["temperature"].view(-1, 1), prm["top_k"].view(-1, 1), prm["top_p"].view(-1, 1),
                          torch.arange(1024, device=DEV))
    for r in range(half):
        got_k, want_k = probs_out[r] > 0, want[r] > 0
        if not torch.equal(got_k, want_k):
            # only the top-p boundary token may differ, where the cumulative
            # probability before it is within 1e-5 of top_p
            diff = (got_k ^ want_k).nonzero().flatten().tolist()
            assert len(diff) == 1, (r, diff)
            sv, si = torch.sort(cfg[r] / prm["temperature"][r], descending=True)
            k = int(prm["top_k"][r]) or 1024
            pr = torch.softmax(sv[:k], 0)
            rank = int((si[:k] == diff[0]).nonzero())
            assert abs(float(pr[:rank].sum()) - float(prm["top_p"][r])) < 1e-5, r
            continue
        torch.testing.assert_close(probs_out[r], want[r], rtol=1e-5, atol=1e-6)
    # greedy rows: the first argmax of the combined logits; twins match
    assert torch.equal(tokens[:half], tokens[half:])
    g = half // 2
    assert torch.equal(tokens[g:half], cfg_out[g:].argmax(-1))
    # sampled rows draw a kept token; row 1 (top_k 1, top_p 0) draws the argmax
    for r in range(g):
        assert probs_out[r, tokens[r]] > 0, r
    assert int(tokens[1]) == int(cfg_out[1].argmax()) == int(cfg[1].argmax())


def test_greedy_rows_without_probabilities_take_the_argmax_only():
    """Greedy rows with no probs_out stop after the argmax.  The same mixed
    batch (half the rows sampled) with and without probs_out, from equal
    seeds and call counts, gives the same tokens and call counts."""
    gen = torch.Generator(device=DEV).manual_seed(3)
    half, V, codec = 16, 2051, 2048
    logits = torch.randn(2 * half, V, device=DEV, generator=gen) * 3
    prm = _params(half, temperature=0.8, top_k=50, top_p=0.9)
    prm["do_sample"][::2] = 0
    runs = []
    for probs in (True, False):
        st = SampleState(half, DEV, seed=11)
        tokens = torch.full((2 * half,), -1, dtype=torch.int64, device=DEV)
        cfg_out = torch.empty(half, V, device=DEV)
        kw = dict(probs_out=torch.empty(half, V, device=DEV)) if probs else {}
        for _ in range(3):  # three calls: the counters advance on both paths
            sample_cfg(logits, tokens, st, codec_size=codec, cfg_out=cfg_out, **kw, **prm)
        torch.cuda.synchronize()
        runs.append((tokens.clone(), st.counters.clone(), cfg_out))
    (ta, ca, cfg), (tb, cb, _) = runs
    assert torch.equal(ta, tb)
    assert torch.equal(ca, cb)
    assert torch.equal(tb[0:half:2], cfg[0::2].argmax(-1))
    assert torch.equal(tb[:half], tb[half:])


def test_draws_follow_the_distribution():
    from scipy.stats import chi2

    V, rows = 64, 4096
    base = torch.linspace(-2, 2, V, device=DEV) + torch.sin(torch.arange(V, device=DEV).float())
    logits = base.expand(rows, V).contiguous()  # B = rows: CFG pairs of identical rows
    half = rows // 2
    prm = _params(half, temperature=1.3, guidance=1.0)
    st = SampleState(half, DEV, seed=123)
    tokens = torch.empty(rows, dtype=torch.int64, device=DEV)
    counts = torch.zeros(V, dtype=torch.int64, device=DEV)
    for _ in range(10):
        sample_cfg(logits, tokens, st, **prm)
        counts += torch.bincount(tokens[:half], minlength=V)
    n = int(counts.sum())
    p = torch.softmax(base / 1.3, 0).double()
    stat = float((((counts.double() - n * p) ** 2) / (n * p)).sum())
    assert chi2.sf(stat, V - 1) > 1e-4, stat
    assert int(st.counters.min()) == int(st.counters.max()) == 10


def test_stream_is_reproducible_and_advances():
    V, half = 300, 8
    gen = torch.Generator(device=DEV).manual_seed(5)
    logits = torch.randn(2 * half, V, device=DEV, generator=gen)
    prm = _params(half, temperature=2.0, guidance=1.5)
    st = SampleState(half, DEV, seed=99)
    out = [torch.empty(2 * half, dtype=torch.int64, device=DEV) for _ in range(4)]
    sample_cfg(logits, out[0], st, **prm)
    sample_cfg(logits, out[1], st, **prm)
    st.reseed(99)
    sample_cfg(logits, out[2], st, **prm)
    st.reseed(100)
    sample_cfg(logits, out[3], st, **prm)
    assert torch.equal(out[0], out[2])
    assert not torch.equal(out[0], out[1]) and not torch.equal(out[0], out[3])


def test_graph_replays_advance_and_match_eager():
    V, half = 2051, 2
    gen = torch.Generator(device=DEV).manual_seed(8)
    logits = torch.randn(2 * half, V, device=DEV, generator=gen)
    prm = _params(half, temperature=1.5, top_k=50, top_p=0.95, guidance=3.0)
    st = SampleState(half, DEV, seed=31)
    tokens = torch.empty(2 * half, dtype=torch.int64, device=DEV)
    eager = []
    for _ in range(6):
        sample_cfg(logits, tokens, st, **prm)
        eager.append(tokens.clone())
    st.reseed(31)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            sample_cfg(logits, tokens, st, **prm)
    torch.cuda.current_stream().wait_stream(s)
    st.reseed(31)  # capture does not run the kernel
    for i in range(6):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(tokens, eager[i]), i
        _ = torch.randn(256, device=DEV).sum().item()  # eager work between replays
    assert len({tuple(t.tolist()) for t in eager}) > 1
