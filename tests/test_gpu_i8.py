"""Parity of the int8 matrix-core path (cfg path 3) for int4 weights, through
the C ABI.  x is carried as two int8 planes per row (u = s_x (hi + lo/254),
about 16 significant bits), so the same-rounding bar (4e-3 against the
oracle with the kernel's folded-norm rounding) and the reference's 1e-2 bar
both apply unchanged; a one-hot x selects a weight column to within 1e-6."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import bz_oracle as O
from tests._util import Int4Case, bf16_tensor, f32, u8_tensor

from breeze_amd import gemv as G

pytestmark = pytest.mark.gpu

TOL = 1e-2
TIGHT = 4e-3
GOLDEN = Path(__file__).resolve().parent / "golden"
P3 = (0, 0, 0, 3)


def _run(c: Int4Case, x_bits, gamma_bits, layout, epi, res_bits=None, cfg=P3, out_dtype=torch.bfloat16):
    x = bf16_tensor(x_bits)
    gamma = bf16_tensor(gamma_bits) if gamma_bits is not None else None
    res = bf16_tensor(res_bits) if res_bits is not None else None
    if layout == "zp":
        return G.gemv(x, c.d_packed, G.W_INT4_ZP, c.N, sc0=c.d_sz, group=c.group, gamma=gamma, epilogue=epi,
                      residual=res, cfg=cfg, out_dtype=out_dtype)
    return G.gemv(x, c.d_packed, G.W_INT4_MIN, c.N, sc0=c.d_s, sc1=c.d_m, group=c.group, gamma=gamma,
                  epilogue=epi, residual=res, cfg=cfg, out_dtype=out_dtype)


def _refs(x_bits, gamma_bits, norm, w_eff, epi, res=None):
    x = O.bf16_bits_to_f32(x_bits)
    if norm:
        g = O.bf16_bits_to_f32(gamma_bits)
        a, b = O.rmsnorm_f32(x, g), O.rmsnorm_folded(x, g)
    else:
        a = b = x
    return O.gemv_ref(a, w_eff, epi, res), O.gemv_ref(b, w_eff, epi, res)


@pytest.mark.parametrize("layout", ["zp", "min"])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 13, 16])
@pytest.mark.parametrize("epi", [0, 1, 2])
@pytest.mark.parametrize("norm", [False, True])
def test_i8_int4_small(layout, M, epi, norm):
    N, K = 272, 768   # ragged: 17 tiles of 16 columns (8.5 for the SiLU half); 6 units per row
    w, gamma, x = O.synth(N, K, M, seed=100 + M * 7 + epi)
    c = Int4Case(w, 128)
    n_out = N // 2 if epi == 1 else N
    res_bits = O.f32_to_bf16_bits(np.random.default_rng(5).standard_normal((M, n_out)).astype(np.float32))
    got = f32(_run(c, x, gamma if norm else None, layout, epi, res_bits if epi == 2 else None))
    w_eff = c.w_zp if layout == "zp" else c.w_min
    ref, ref_same = _refs(x, gamma, norm, w_eff, epi, O.bf16_bits_to_f32(res_bits) if epi == 2 else None)
    assert O.rel_err(got, ref) <= TOL
    assert O.rel_err(got, ref_same) <= TIGHT


@pytest.mark.parametrize("M", [1, 2])
def test_i8_c1(M):
    w, gamma, x = O.synth(2048, 2048, M, seed=0)
    c = Int4Case(w, 128, symmetric=True)
    got = f32(_run(c, x, gamma, "zp", G.EPI_NONE))
    ref, ref_same = _refs(x, gamma, True, c.w_zp, O.EPI_NONE)
    assert O.rel_err(got, ref) <= TOL and O.rel_err(got, ref_same) <= TIGHT


def test_i8_one_hot_selects_column():
    N, K, group = 64, 512, 128
    rng = np.random.default_rng(9)
    q = rng.integers(0, 16, (N, K), dtype=np.uint8)
    s = (2.0 ** rng.integers(-8, -4, (N, K // group))).astype(np.float32)
    z = (rng.integers(-64, 64, (N, K // group)) * 2.0 ** -9).astype(np.float32)
    sz = O.scales_zeros(s, z)
    w_eff = O.dequant_int4_zp(q, sz, group)
    d_w, d_sz = u8_tensor(O.pack_nibbles_even_low(q)), bf16_tensor(sz)
    ks = list(range(0, K, 37)) + [K - 1]
    x = np.zeros((len(ks), K), np.float32)
    x[np.arange(len(ks)), ks] = 1.0
    got = f32(G.gemv(bf16_tensor(O.f32_to_bf16_bits(x)), d_w, G.W_INT4_ZP, N, sc0=d_sz, group=group,
                     out_dtype=torch.float32, cfg=P3))
    for i, k in enumerate(ks):
        np.testing.assert_allclose(got[i], w_eff[:, k], rtol=1e-6, atol=1e-9)


@pytest.mark.parametrize("depth,nw,tiles", [(2, 1, 1), (2, 7, 3), (4, 3, 0), (4, 8, 2), (8, 8, 1), (8, 5, 0)])
@pytest.mark.parametrize("epi", [1, 2])
def test_i8_launch_shapes_agree(depth, nw, tiles, epi):
    N, K, M = 512, 2560, 3
    w, gamma, x = O.synth(N, K, M, seed=4)
    c = Int4Case(w)
    n_out = N // 2 if epi == 1 else N
    res_bits = O.f32_to_bf16_bits(np.random.default_rng(8).standard_normal((M, n_out)).astype(np.float32))
    res = res_bits if epi == 2 else None
    got = f32(_run(c, x, gamma, "zp", epi, res, cfg=(depth, nw, tiles, 3)))
    base = f32(_run(c, x, gamma, "zp", epi, res))
    ref, ref_same = _refs(x, gamma, True, c.w_zp, epi, O.bf16_bits_to_f32(res_bits) if epi == 2 else None)
    assert O.rel_err(got, ref_same) <= TIGHT
    assert O.rel_err(got, base) <= TIGHT


def test_i8_rows_sliced_by_lds():
    """K = 10240 leaves room for fewer than 16 rows per launch: M = 20 runs in
    several launches and every row is right."""
    N, K, M = 256, 10240, 20
    w, gamma, x = O.synth(N, K, M, seed=12)
    c = Int4Case(w)
    got = f32(_run(c, x, gamma, "zp", G.EPI_NONE))
    ref, ref_same = _refs(x, gamma, True, c.w_zp, O.EPI_NONE)
    assert O.rel_err(got, ref) <= TOL and O.rel_err(got, ref_same) <= TIGHT
    for m in range(M):
        assert O.rel_err(got[m], ref_same[m]) <= TIGHT, m


@pytest.mark.parametrize("name", ["int4_asym_g128", "int4_sym_g128"])
def test_i8_golden(name):
    f = np.load(GOLDEN / f"{name}.npz")
    n, k, m, group, sym = (int(v) for v in f["meta"])
    d_p = u8_tensor(f["packed_even_low"])
    x, g = bf16_tensor(f["x"]), bf16_tensor(f["gamma"])
    sz = bf16_tensor(f["scales_zeros"])
    out = G.gemv(x, d_p, G.W_INT4_ZP, n, sc0=sz, group=group, gamma=g, out_dtype=torch.float32, cfg=P3)
    assert O.rel_err(f32(out), f["out_norm_none"]) <= TOL
    out = G.gemv(x, d_p, G.W_INT4_ZP, n, sc0=sz, group=group, gamma=g, epilogue=G.EPI_SILU_GATE, cfg=P3)
    assert O.rel_err(f32(out), f["out_norm_silu"]) <= TOL
    out = G.gemv(x, d_p, G.W_INT4_MIN, n, sc0=bf16_tensor(f["scale_bits"]), sc1=bf16_tensor(f["min_bits"]),
                 group=group, cfg=P3)
    assert O.rel_err(f32(out), f["out_min_none"]) <= TOL


def test_i8_zero_row_and_extremes():
    """An all-zero x row (scale floor) gives the residual back.  A row with one
    value 30000x its neighbours: only its own 128-k unit shares the coarse
    scale (neighbour step s_x/254 ~ 0.009 against values ~0.01, summing to
    ~1e-4 of the output), the other units keep their own fine scales."""
    N, K, M = 128, 512, 2
    w, _, _ = O.synth(N, K, M, seed=13)
    c = Int4Case(w)
    x = np.zeros((M, K), np.float32)
    x[1] = np.random.default_rng(14).standard_normal(K).astype(np.float32) * 0.01
    x[1, 7] = 300.0
    xb = O.f32_to_bf16_bits(x)
    res_bits = O.f32_to_bf16_bits(np.random.default_rng(15).standard_normal((M, N)).astype(np.float32))
    got = f32(_run(c, xb, None, "zp", G.EPI_RESIDUAL, res_bits, out_dtype=torch.float32))
    np.testing.assert_array_equal(got[0], O.bf16_bits_to_f32(res_bits)[0])
    ref = O.gemv_ref(O.bf16_bits_to_f32(xb), c.w_zp, O.EPI_RES, O.bf16_bits_to_f32(res_bits))
    assert O.rel_err(got[1], ref[1]) <= 1e-3


def test_i8_needs_int4_group_128():
    w, gamma, x = O.synth(64, 512, 1, seed=6)
    c = Int4Case(w, 64)
    with pytest.raises(RuntimeError, match="exceeds what this build supports"):
        _run(c, x, gamma, "zp", G.EPI_NONE)
    with pytest.raises(RuntimeError, match="exceeds what this build supports"):
        G.gemv(bf16_tensor(x), torch.zeros(64, 512, dtype=torch.uint8, device="cuda"), G.W_FP8, 64,
               sc0=torch.ones(64, device="cuda"), cfg=P3)
