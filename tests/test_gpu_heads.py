"""fp32 heads through the C ABI against the oracle (float64), on the GPU.
Bar: 1e-5 of the largest output (fp32 products and sums over K <= 2560)."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

from oracle import bz_oracle as O
from tests._util import f32

from breeze_amd import heads as Hd

pytestmark = pytest.mark.gpu

TOL = 1e-5
DEV = "cuda"


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 9])
@pytest.mark.parametrize("K,N", [(1024, 2051), (2048, 2052), (2560, 8192), (64, 7)])
def test_head_f32_matches_oracle(M, K, N):
    rng = np.random.default_rng(M * 31 + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    got = f32(Hd.head_f32(torch.from_numpy(x).to(DEV), torch.from_numpy(w).to(DEV)))
    assert O.rel_err(got, O.linear_f32_ref(x, w)) <= TOL


def test_head_f32_device_index_selects_matrix_and_out_of_range_is_zero():
    rng = np.random.default_rng(3)
    C, N, K = 5, 300, 256
    w = rng.standard_normal((C, N, K)).astype(np.float32)
    x = rng.standard_normal((2, K)).astype(np.float32)
    wd, xd = torch.from_numpy(w).to(DEV), torch.from_numpy(x).to(DEV)
    for pos in (1, 3, 5):
        idx = torch.tensor([pos], device=DEV)
        got = f32(Hd.head_f32(xd, wd, index=idx, index_offset=-1))
        assert O.rel_err(got, O.linear_f32_ref(x, w[pos - 1])) <= TOL
    for pos in (0, 6, -3):
        got = f32(Hd.head_f32(xd, wd, index=torch.tensor([pos], device=DEV), index_offset=-1))
        assert not got.any()


def test_fp32_linear_matches_torch_fp32():
    torch.manual_seed(0)
    lin = nn.Linear(2048, 2052, bias=False)
    head = Hd.Fp32Linear(lin)
    x = torch.randn(2, 1, 2048).to(torch.bfloat16)
    got = head(x.to(DEV))
    assert got.dtype == torch.float32 and got.shape == (2, 1, 2052)
    ref = O.linear_f32_ref(x.float().reshape(2, 2048).numpy(), lin.weight.detach().numpy())
    assert O.rel_err(f32(got).reshape(2, 2052), ref) <= TOL


class _CodebooksHead(nn.Module):
    """Same parameters as models/breeze.py:590-596 (weight [C - 1, hidden, vocab])."""

    def __init__(self, hidden, num_codebooks, vocab):
        super().__init__()
        self.num_codebooks = num_codebooks
        self.weight = nn.Parameter(torch.randn(num_codebooks - 1, hidden, vocab) * 0.02)


@pytest.mark.parametrize("with_position", [False, True])
def test_fp32_codebooks_head(with_position):
    torch.manual_seed(1)
    ref_head = _CodebooksHead(1024, 16, 2051)
    head = Hd.Fp32CodebooksHead(ref_head)
    B, L = 2, (1 if with_position else 15)
    hidden = torch.randn(B, L, 1024).to(torch.bfloat16)
    cp = torch.tensor([7]) if with_position else None
    got = head(hidden.to(DEV), None if cp is None else cp.to(DEV))
    ref = O.codebooks_head_ref(hidden.float().numpy(), ref_head.weight.detach().numpy(),
                               None if cp is None else cp.numpy())
    assert got.shape == (B, L, 2051)
    assert O.rel_err(f32(got), ref) <= TOL


def test_codebooks_head_graph_replays_follow_device_position():
    """Captured once; the cache position changes between replays (as in the
    depth decoder's graph) and every replay uses its codebook."""
    torch.manual_seed(2)
    ref_head = _CodebooksHead(1024, 16, 2051)
    head = Hd.Fp32CodebooksHead(ref_head)
    hidden = torch.randn(2, 1, 1024, device=DEV)
    cp = torch.ones(1, dtype=torch.int64, device=DEV)
    out = torch.empty(2, 1, 2051, device=DEV)
    head(hidden, cp)
    torch.cuda.synchronize()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st):
        with torch.cuda.graph(g, stream=st):
            out.copy_(head(hidden, cp))
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    w = ref_head.weight.detach().numpy()
    for p in (1, 15, 4, 9):
        cp.fill_(p)
        g.replay()
        torch.cuda.synchronize()
        ref = O.codebooks_head_ref(f32(hidden), w, np.array([p]))
        assert O.rel_err(f32(out), ref) <= TOL, p


def test_install_fp32_heads():
    class _Model(nn.Module):
        def __init__(self):
            super().__init__()
            self.lm_head = nn.Linear(256, 2052, bias=False)
            self.depth_decoder = nn.Module()
            self.depth_decoder.codebooks_head = _CodebooksHead(128, 4, 2051)

    m = _Model()
    assert Hd.install_fp32_heads(m) == 2
    assert isinstance(m.lm_head, Hd.Fp32Linear)
    assert isinstance(m.depth_decoder.codebooks_head, Hd.Fp32CodebooksHead)
    assert Hd.install_fp32_heads(m) == 0
