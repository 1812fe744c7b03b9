"""The sharded decomposition of the decode GEMVs, on one GPU.

A G-way tensor-parallel decoder layer would run the same kernels on smaller
shapes:
  * column-parallel gate|up: shard i holds the gate rows AND the matching up
    rows of its output slice ([gate_i; up_i]), so the SiLU-gate epilogue
    stays local and the output slices simply concatenate;
  * row-parallel down / o_proj: shard i holds a K slice (whole quantization
    groups) and writes fp32 partials; one all-reduce sums them and the
    residual is added after the sum.
These tests run every shard on the one GPU and check that the pieces
reassemble the unsharded result (and the oracle) within the 1e-2 tolerance
of max|out-ref|/max|ref|.  No collective or rank code is involved: the sum
stands in for the all-reduce."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import bz_oracle as O
from tests._util import Int4Case, bf16_tensor

pytestmark = pytest.mark.gpu


def _x(M, K, seed):
    return O.f32_to_bf16_bits(np.random.default_rng(seed).standard_normal((M, K)).astype(np.float32))


@pytest.mark.parametrize("M", [1, 2])
@pytest.mark.parametrize("shards", [2, 8])
def test_column_parallel_gate_up(M, shards):
    from breeze_amd import gemv as G

    K, NO = 2560, 2048                      # N_out = 2048: [gate (2048 rows); up (2048 rows)]
    rng = np.random.default_rng(100 + shards)
    w = (rng.standard_normal((2 * NO, K)) * 0.02).astype(np.float32)
    gamma = O.f32_to_bf16_bits((1 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    xb = _x(M, K, 7)
    full = Int4Case(w, 128, symmetric=True)
    x, g = bf16_tensor(xb), bf16_tensor(gamma)
    want = G.gemv(x, full.d_packed, G.W_INT4_ZP, 2 * NO, sc0=full.d_sz, gamma=g, epilogue=G.EPI_SILU_GATE)
    ref = O.gemv_ref(O.rmsnorm_f32(O.bf16_bits_to_f32(xb), O.bf16_bits_to_f32(gamma)), full.w_zp, O.EPI_SILU)
    n = NO // shards
    parts = []
    for i in range(shards):
        rows = np.r_[i * n:(i + 1) * n, NO + i * n:NO + (i + 1) * n]   # [gate_i; up_i]
        # the shard's rows quantize exactly as in the full matrix (groups run along K)
        sh = Int4Case(w[rows], 128, symmetric=True)
        np.testing.assert_array_equal(sh.packed, full.packed[rows])
        parts.append(G.gemv(x, sh.d_packed, G.W_INT4_ZP, 2 * n, sc0=sh.d_sz, gamma=g, epilogue=G.EPI_SILU_GATE))
    got = torch.cat(parts, dim=1)
    torch.cuda.synchronize()
    assert O.rel_err(got.float().cpu().numpy(), ref) <= 1e-2
    assert O.rel_err(got.float().cpu().numpy(), want.float().cpu().numpy()) <= 1e-2


@pytest.mark.parametrize("M", [1, 2])
@pytest.mark.parametrize("shards", [2, 8])
def test_row_parallel_down_with_residual(M, shards):
    from breeze_amd import gemv as G

    N, K = 2560, 8192
    rng = np.random.default_rng(200 + shards)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    xb, rb = _x(M, K, 8), _x(M, N, 9)
    full = Int4Case(w, 128, symmetric=True)
    x, res = bf16_tensor(xb), bf16_tensor(rb)
    want = G.gemv(x, full.d_packed, G.W_INT4_ZP, N, sc0=full.d_sz, epilogue=G.EPI_RESIDUAL, residual=res)
    ref = O.gemv_ref(O.bf16_bits_to_f32(xb), full.w_zp, O.EPI_RES, O.bf16_bits_to_f32(rb))
    k = K // shards
    total = torch.zeros(M, N, device="cuda", dtype=torch.float32)
    for i in range(shards):
        ks = slice(i * k, (i + 1) * k)
        # K slice of whole groups: packed bytes [k/2 ...], scales_zeros rows [k/128 ...]
        pw = full.d_packed[:, i * k // 2:(i + 1) * k // 2].contiguous()
        psz = full.d_sz[i * k // 128:(i + 1) * k // 128].contiguous()
        total += G.gemv(x[:, ks].contiguous(), pw, G.W_INT4_ZP, N, sc0=psz, out_dtype=torch.float32)
    got = (total + res.float()).cpu().numpy()      # the all-reduce, then the residual
    torch.cuda.synchronize()
    assert O.rel_err(got, ref) <= 1e-2
    assert O.rel_err(got, want.float().cpu().numpy()) <= 1e-2


def test_row_shards_sum_exactly_in_fp32():
    """With fp32 partials and shards of whole groups, the shard sums differ
    from the unsharded fp32 result only by fp32 reassociation."""
    from breeze_amd import gemv as G

    N, K = 2048, 4096
    rng = np.random.default_rng(300)
    full = Int4Case((rng.standard_normal((N, K)) * 0.02).astype(np.float32), 128, symmetric=True)
    xb = _x(1, K, 10)
    x = bf16_tensor(xb)
    whole = G.gemv(x, full.d_packed, G.W_INT4_ZP, N, sc0=full.d_sz, out_dtype=torch.float32)
    parts = [G.gemv(x[:, i * 1024:(i + 1) * 1024].contiguous(),
                    full.d_packed[:, i * 512:(i + 1) * 512].contiguous(), G.W_INT4_ZP, N,
                    sc0=full.d_sz[i * 8:(i + 1) * 8].contiguous(), out_dtype=torch.float32) for i in range(4)]
    s = sum(parts)
    torch.cuda.synchronize()
    scale = whole.abs().max().item()
    assert (s - whole).abs().max().item() <= 1e-5 * scale * K ** 0.5
