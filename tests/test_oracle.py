"""Pins of the CPU oracle (oracle/bz_oracle.py), CPU only.

Each check is chosen so that a plausible mistake in the oracle (a dropped
term, a wrong sign or offset, a swapped nibble, a transposed scale table)
fails it: closed forms, exactly representable inputs, brute-force scalar
loops, invariants, an independent library (torch's CPU float8_e4m3fn and
bfloat16 casts) and the committed golden fixtures.  The last test plants
such mistakes in copies of oracle functions and checks that the pins catch
them.
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import bz_oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"


# ---------------------------------------------------------------------------
# bfloat16 rounding
# ---------------------------------------------------------------------------


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    a = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(3.0),
        rng.standard_normal(2000).astype(np.float32) * np.float32(1e-30),
        np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, 3.4e38, -3.4e38, 1e-45], dtype=np.float32),
    ])
    # exact ties: bit 15 set, bits 0..14 clear (round half to even)
    ties = (rng.integers(0, 1 << 16, 2000).astype(np.uint32) << 16 | 0x8000).astype(np.uint32)
    ties = ties[np.isfinite(ties.view(np.float32))]
    a = np.concatenate([a, ties.view(np.float32)])
    want = torch.from_numpy(a).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.f32_to_bf16_bits(a), want)


def test_bf16_nan_stays_nan():
    bits = O.f32_to_bf16_bits(np.array([np.nan, -np.nan], dtype=np.float32))
    assert np.all(np.isnan(O.bf16_bits_to_f32(bits)))


# ---------------------------------------------------------------------------
# OCP e4m3 ("fn")
# ---------------------------------------------------------------------------


def test_e4m3fn_decode_closed_forms():
    t = O.e4m3fn_decode_table()
    assert t[0x00] == 0.0 and t[0x80] == 0.0 and math.copysign(1, t[0x80]) == -1
    assert t[0x38] == 1.0 and t[0xB8] == -1.0          # exponent field 7 = bias
    assert t[0x7E] == 448.0 and t[0xFE] == -448.0      # largest finite
    assert t[0x01] == 2.0 ** -9                        # smallest subnormal
    assert t[0x07] == 7 * 2.0 ** -9                    # largest subnormal
    assert t[0x08] == 2.0 ** -6                        # smallest normal
    assert np.isnan(t[0x7F]) and np.isnan(t[0xFF])     # the only NaNs
    assert np.sum(np.isnan(t)) == 2
    pos = t[:0x7F]
    assert np.all(np.diff(pos) > 0)                    # codes 0..126 increase


def test_e4m3fn_decode_matches_torch():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    want = codes.view(torch.float8_e4m3fn).float().numpy()
    got = O.e4m3fn_decode(np.arange(256, dtype=np.uint8))
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok], want[ok])


def test_e4m3fn_decode_fixture():
    f = np.load(GOLDEN / "e4m3fn_table.npz")
    got = O.e4m3fn_decode(f["codes"])
    assert np.array_equal(np.isnan(got), np.isnan(f["values"]))
    ok = ~np.isnan(got)
    assert np.array_equal(got[ok], f["values"][ok])


def test_e4m3fn_encode_matches_torch_dense():
    rng = np.random.default_rng(1)
    pos = O.e4m3fn_decode_table()[:0x7F].astype(np.float64)
    mids = ((pos[1:] + pos[:-1]) / 2).astype(np.float32)             # exact ties
    near = np.concatenate([np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1e9))])
    a = np.concatenate([
        rng.uniform(-448, 448, 40000).astype(np.float32),
        rng.uniform(-0.02, 0.02, 20000).astype(np.float32),            # subnormal range
        mids, -mids, near, -near, pos.astype(np.float32), -pos.astype(np.float32),
        np.array([0.0, -0.0, 448.0, -448.0, 1e-12, -1e-12], dtype=np.float32),
    ])
    a = np.clip(a, -448, 448).astype(np.float32)
    want = torch.from_numpy(a).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = O.e4m3fn_encode(a)
    # torch keeps the sign of a value that rounds to zero; so does the oracle
    assert np.array_equal(got, want)


def test_e4m3fn_encode_ties_to_even():
    t = O.e4m3fn_decode_table()
    # midpoint of codes 0x38 (1.0) and 0x39 (1.125): even code 0x38 wins
    assert O.e4m3fn_encode(np.float32(1.0625)) == 0x38
    # midpoint of 0x39 and 0x3A: even code 0x3A wins
    assert O.e4m3fn_encode(np.float32((t[0x39] + t[0x3A]) / 2)) == 0x3A


def test_e4m3fn_encode_rejects_unclamped():
    with pytest.raises(ValueError):
        O.e4m3fn_encode(np.float32(449.0))


# ---------------------------------------------------------------------------
# int4 quantizers
# ---------------------------------------------------------------------------


def test_int4_asym_constant_group_hits_scale_floor():
    w = np.full((2, 128), 0.3, dtype=np.float32)
    q, s, lo, z = O.quantize_int4_asym(w, 128)
    assert np.all(q == 0)
    assert np.all(s == np.float32(1e-8))
    assert np.all(lo == np.float32(0.3))
    assert np.all(z == np.float32(0.3) + np.float32(8.0) * np.float32(1e-8))


def test_int4_asym_on_grid_weights_recovered_exactly():
    rng = np.random.default_rng(2)
    n, k, g = 6, 512, 128
    s_true = np.float32(2.0 ** -6)
    lo_true = rng.integers(-64, 0, (n, k // g)).astype(np.float32) * s_true
    q_true = rng.integers(0, 16, (n, k)).astype(np.uint8)
    q_true[:, ::g] = 0          # every group spans the full 0..15 range,
    q_true[:, 1::g] = 15        # so min and max recover lo and s exactly
    w = np.repeat(lo_true, g, axis=1) + q_true.astype(np.float32) * s_true
    q, s, lo, z = O.quantize_int4_asym(w, g)
    assert np.array_equal(q, q_true)
    assert np.all(s == s_true)
    assert np.array_equal(lo, lo_true)
    assert np.array_equal(z, lo_true + np.float32(8) * s_true)


def test_int4_asym_rounds_half_to_even():
    w = np.zeros((1, 32), dtype=np.float32)
    w[0, 0], w[0, 1] = 0.0, 15.0        # lo = 0, s = 1
    w[0, 2:6] = [0.5, 1.5, 2.5, 14.5]
    q, s, _, _ = O.quantize_int4_asym(w, 32)
    assert s[0, 0] == 1.0
    assert list(q[0, 2:6]) == [0, 2, 2, 14]


def _asym_scalar(w, g):
    """Element-by-element restatement with float32 scalars (brute force)."""
    n, k = w.shape
    q = np.zeros((n, k), np.uint8)
    s = np.zeros((n, k // g), np.float32)
    for r in range(n):
        for j in range(k // g):
            blk = [np.float32(v) for v in w[r, j * g:(j + 1) * g]]
            lo, hi = min(blk), max(blk)
            sc = max(np.float32((hi - lo) / np.float32(15)), np.float32(1e-8))
            s[r, j] = sc
            for i, v in enumerate(blk):
                t = np.float32((v - lo) / sc)
                q[r, j * g + i] = min(max(int(np.rint(t)), 0), 15)
    return q, s


def test_int4_asym_matches_scalar_loop():
    w, _, _ = O.synth(3, 256, 1, seed=3)
    q, s, _, _ = O.quantize_int4_asym(w, 64)
    q2, s2 = _asym_scalar(w, 64)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)


def test_int4_dequant_error_bounded_by_half_step():
    w, _, _ = O.synth(16, 1024, 1, seed=4)
    q, s, lo, z = O.quantize_int4_asym(w, 128)
    w_eff = O.dequant_int4_zp(q, O.scales_zeros(s, z), 128)
    sb = np.repeat(O.round_bf16(s), 128, axis=1)
    # half a step, plus the bf16 rounding of s (<= 2^-9 |s| per unit of |q-8| <= 8)
    # and of z (<= 2^-9 |z|)
    bound = 0.5 * sb + 8 * 2.0 ** -8 * sb + 2.0 ** -8 * np.repeat(np.abs(z), 128, axis=1) + 1e-9
    assert np.all(np.abs(w_eff - w) <= bound)


def test_int4_sym_properties():
    w, _, _ = O.synth(8, 512, 1, seed=5)
    q, s, z = O.quantize_int4_sym(w, 128)
    assert np.all(z == 0)
    assert q.min() >= 1 and q.max() <= 15           # |w| <= 7 s -> q - 8 in [-7, 7]
    w_eff = (q.astype(np.float32) - 8) * np.repeat(s, 128, axis=1)
    assert np.all(np.abs(w_eff - w) <= 0.5 * np.repeat(s, 128, axis=1) * (1 + 1e-6))
    # on-grid weights (absmax = 7 s) come back exactly
    s0 = np.float32(2.0 ** -7)
    qt = np.random.default_rng(6).integers(1, 16, (2, 128)).astype(np.uint8)
    qt[:, 0] = 15
    q2, s2, _ = O.quantize_int4_sym((qt.astype(np.float32) - 8) * s0, 128)
    assert np.array_equal(q2, qt) and np.all(s2 == s0)


# ---------------------------------------------------------------------------
# nibble packing and the scales_zeros table
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("k", [0, 1, 2, 7, 254, 255])
def test_single_nibble_positions(k):
    for v in (1, 9, 15):
        q = np.zeros((2, 256), np.uint8)
        q[1, k] = v
        ev, od = O.pack_nibbles_even_low(q), O.pack_nibbles_odd_low(q)
        assert np.count_nonzero(ev) == 1 and np.count_nonzero(od) == 1
        assert ev[1, k // 2] == (v << (4 * (k % 2)))         # even k -> low nibble
        assert od[1, k // 2] == (v << (4 * (1 - k % 2)))     # odd k -> low nibble


def test_pack_unpack_round_trip():
    q = np.random.default_rng(7).integers(0, 16, (5, 96)).astype(np.uint8)
    assert np.array_equal(O.unpack_nibbles_even_low(O.pack_nibbles_even_low(q)), q)
    assert np.array_equal(O.unpack_nibbles_odd_low(O.pack_nibbles_odd_low(q)), q)
    swapped = q.reshape(5, -1, 2)[:, :, ::-1].reshape(5, -1)
    assert np.array_equal(O.pack_nibbles_even_low(q), O.pack_nibbles_odd_low(swapped))


def test_scales_zeros_layout():
    rng = np.random.default_rng(8)
    s = rng.standard_normal((6, 4)).astype(np.float32)
    z = rng.standard_normal((6, 4)).astype(np.float32)
    sz = O.scales_zeros(s, z)
    assert sz.shape == (4, 6, 2) and sz.dtype == np.uint16
    for n in range(6):
        for g in range(4):
            assert sz[g, n, 0] == O.f32_to_bf16_bits(s[n, g])
            assert sz[g, n, 1] == O.f32_to_bf16_bits(z[n, g])
    # and the same table as torch.stack([s.t(), z.t()], -1).to(bfloat16)
    want = torch.stack([torch.from_numpy(s).t(), torch.from_numpy(z).t()], -1).to(torch.bfloat16)
    assert np.array_equal(sz, want.view(torch.int16).numpy().view(np.uint16))


def test_zp_and_min_forms_agree():
    w, _, _ = O.synth(8, 256, 1, seed=9)
    q, s, lo, z = O.quantize_int4_asym(w, 128)
    a = O.dequant_int4_zp(q, O.scales_zeros(s, z), 128)
    b = O.dequant_int4_min(q, O.f32_to_bf16_bits(s), O.f32_to_bf16_bits(lo), 128)
    # identical up to the separate bf16 roundings of z = lo + 8 s and of lo
    tol = 2.0 ** -8 * (np.abs(np.repeat(z, 128, 1)) + np.abs(np.repeat(lo, 128, 1)) + 8 * np.repeat(s, 128, 1))
    assert np.all(np.abs(a - b) <= tol + 1e-9)


def test_pack_int4_fused_semantics():
    w, _, _ = O.synth(4, 256, 1, seed=10)
    packed, s_bits, m_bits = O.pack_int4_fused(w)
    q = O.unpack_nibbles_even_low(packed)
    w_eff = O.dequant_int4_min(q, s_bits, m_bits, 128)
    s = np.repeat(O.bf16_bits_to_f32(s_bits), 128, 1)
    assert np.all(np.abs(w_eff - w) <= 0.5 * s + 2.0 ** -8 * (np.abs(w) + 16 * s))


# ---------------------------------------------------------------------------
# fp8 quantizers
# ---------------------------------------------------------------------------


def test_fp8_row_amax_maps_to_448():
    w, _, _ = O.synth(16, 256, 1, seed=11)
    codes, scale = O.quantize_fp8_linear(w)
    amax_pos = np.abs(w).argmax(axis=1)
    for r in range(16):
        assert codes[r, amax_pos[r]] & 0x7F == 0x7E
        assert (codes[r, amax_pos[r]] >> 7) == (w[r, amax_pos[r]] < 0)
    assert np.allclose(scale, np.abs(w).max(axis=1) / 448.0, rtol=1e-7, atol=0)


def test_fp8_floors():
    z = np.zeros((2, 64), np.float32)
    c1, s1 = O.quantize_fp8_linear(z)
    c2, s2 = O.pack_fp8(z)
    assert np.all(c1 == 0) and np.all(c2 == 0)
    assert np.all(s1 == np.float32(np.float32(1e-12) / np.float32(448)))
    assert np.all(s2 == np.float32(np.float32(1e-8) / np.float32(448)))


def test_fp8_dequant_relative_error():
    w, _, _ = O.synth(8, 512, 1, seed=12)
    codes, scale = O.quantize_fp8_linear(w)
    w_eff = O.dequant_fp8(codes, scale)
    # e4m3: 3 mantissa bits -> relative error <= 2^-4 for normals; absolute
    # error <= half the subnormal step (2^-10 * scale) below 2^-6 * scale
    err = np.abs(w_eff - w)
    bound = np.maximum(2.0 ** -4 * np.abs(w), 2.0 ** -10 * scale[:, None]) * (1 + 1e-6)
    assert np.all(err <= bound)


# ---------------------------------------------------------------------------
# RMSNorm
# ---------------------------------------------------------------------------


def test_rmsnorm_matches_float64_loop():
    _, gamma, x = O.synth(1, 64, 3, seed=13)
    xf, gf = O.bf16_bits_to_f32(x), O.bf16_bits_to_f32(gamma)
    got = O.rmsnorm_f32(xf, gf, 1e-6)
    for m in range(3):
        ms = sum(float(v) ** 2 for v in xf[m]) / 64
        inv = 1 / math.sqrt(ms + 1e-6)
        want = [float(xf[m, k]) * inv * float(gf[k]) for k in range(64)]
        assert np.allclose(got[m], want, rtol=2e-7, atol=0)


def test_rmsnorm_invariants():
    rng = np.random.default_rng(14)
    x = rng.standard_normal((2, 512)).astype(np.float32)
    ones = np.ones(512, np.float32)
    y = O.rmsnorm_f32(x, ones, 0.0)
    assert np.allclose((y.astype(np.float64) ** 2).mean(axis=1), 1.0, rtol=1e-6)
    assert np.allclose(O.rmsnorm_f32(4 * x, ones, 0.0), y, rtol=1e-6)     # scale invariant
    g = rng.standard_normal(512).astype(np.float32)
    assert np.allclose(O.rmsnorm_f32(x, g, 0.0), y * g, rtol=1e-6)        # gamma is elementwise


def test_rmsnorm_roundings_bracket_the_fp32_form():
    _, gamma, x = O.synth(1, 2560, 2, seed=15)
    xf, gf = O.bf16_bits_to_f32(x), O.bf16_bits_to_f32(gamma)
    ref = O.rmsnorm_f32(xf, gf)
    for f in (O.rmsnorm_bf16, O.rmsnorm_folded, O.rmsnorm_model):
        v = f(xf, gf)
        assert np.all(np.abs(v - ref) <= 2.0 ** -7 * np.abs(ref) + 1e-30), f.__name__
    # rmsnorm_bf16 is a single rounding of the fp32 form
    assert np.array_equal(O.rmsnorm_bf16(xf, gf), O.round_bf16(ref))


# ---------------------------------------------------------------------------
# GEMV and epilogues
# ---------------------------------------------------------------------------


def test_gemv_matches_brute_force():
    rng = np.random.default_rng(16)
    x = rng.standard_normal((2, 12))
    w = rng.standard_normal((6, 12))
    res = rng.standard_normal((2, 6))
    rs = rng.uniform(0.5, 2.0, 6)
    acc = [[sum(x[m, k] * w[n, k] for k in range(12)) for n in range(6)] for m in range(2)]
    acc = np.array(acc)
    assert np.allclose(O.gemv_ref(x, w), acc, rtol=1e-12)
    assert np.allclose(O.gemv_ref(x, w, O.EPI_RES, res), acc + res, rtol=1e-12)
    assert np.allclose(O.gemv_ref(x, w, row_scale=rs), acc * rs, rtol=1e-12)
    g, u = acc[:, :3], acc[:, 3:]
    silu = g / (1 + np.exp(-g))
    assert np.allclose(O.gemv_ref(x, w, O.EPI_SILU), silu * u, rtol=1e-12)
    # the fp8 row scale applies before the SiLU, not after
    g, u = (acc * rs)[:, :3], (acc * rs)[:, 3:]
    assert np.allclose(O.gemv_ref(x, w, O.EPI_SILU, row_scale=rs), g / (1 + np.exp(-g)) * u, rtol=1e-12)


def test_gemv_linearity_one_hot_zero():
    rng = np.random.default_rng(17)
    w = rng.standard_normal((10, 32))
    x1, x2 = rng.standard_normal((1, 32)), rng.standard_normal((1, 32))
    assert np.allclose(O.gemv_ref(2 * x1 - 3 * x2, w), 2 * O.gemv_ref(x1, w) - 3 * O.gemv_ref(x2, w))
    e = np.zeros((1, 32))
    e[0, 5] = 1
    assert np.array_equal(O.gemv_ref(e, w)[0], w[:, 5])
    res = rng.standard_normal((1, 10))
    assert np.array_equal(O.gemv_ref(x1, np.zeros((10, 32)), O.EPI_RES, res), res)


def test_silu_closed_forms():
    assert O.silu(0.0) == 0.0
    assert abs(O.silu(30.0) - 30.0) < 1e-10
    assert abs(O.silu(-30.0)) < 1e-11
    assert abs(O.silu(1.0) - 1 / (1 + math.exp(-1))) < 1e-15


def test_rel_err():
    assert O.rel_err([1.0, 2.0], [1.0, 2.0]) == 0.0
    assert O.rel_err([1.0, 2.5], [1.0, 2.0]) == 0.25


def test_synth_distribution():
    w, gamma, x = O.synth(256, 1024, 4, seed=0)
    assert abs(w.std() - 0.02) < 5e-4 and abs(w.mean()) < 5e-4
    g = O.bf16_bits_to_f32(gamma)
    assert abs(g.mean() - 1) < 0.02 and abs(g.std() - 0.1) < 0.01
    xf = O.bf16_bits_to_f32(x)
    assert abs(xf.std() - 1) < 0.02


# ---------------------------------------------------------------------------
# golden fixtures
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("name", ["int4_asym_g128", "int4_sym_g128", "int4_asym_g32"])
def test_int4_golden(name):
    f = np.load(GOLDEN / f"{name}.npz")
    n, k, m, group, sym = (int(v) for v in f["meta"])
    if sym:
        q, s, z = O.quantize_int4_sym(f["w"], group)
    else:
        q, s, lo, z = O.quantize_int4_asym(f["w"], group)
        assert np.array_equal(lo, f["lo"])
    assert np.array_equal(q, f["q"]) and np.array_equal(s, f["s"]) and np.array_equal(z, f["z"])
    assert np.array_equal(O.pack_nibbles_even_low(q), f["packed_even_low"])
    assert np.array_equal(O.pack_nibbles_odd_low(q), f["packed_odd_low"])
    sz = O.scales_zeros(s, z)
    assert np.array_equal(sz, f["scales_zeros"])
    assert np.array_equal(O.dequant_int4_zp(q, sz, group), f["w_eff_zp"])
    assert np.array_equal(O.dequant_int4_min(q, f["scale_bits"], f["min_bits"], group), f["w_eff_min"])
    xf, gf = O.bf16_bits_to_f32(f["x"]), O.bf16_bits_to_f32(f["gamma"])
    xn = O.rmsnorm_f32(xf, gf)
    assert np.array_equal(O.gemv_ref(xn, f["w_eff_zp"]).astype(np.float32), f["out_norm_none"])
    assert np.array_equal(O.gemv_ref(xn, f["w_eff_zp"], O.EPI_SILU).astype(np.float32), f["out_norm_silu"])


def test_fp8_golden():
    f = np.load(GOLDEN / "fp8_row.npz")
    codes, scale = O.quantize_fp8_linear(f["w"])
    assert np.array_equal(codes, f["codes"]) and np.array_equal(scale, f["scale"])
    c8, s8 = O.pack_fp8(f["w"])
    assert np.array_equal(c8, f["codes_fused"]) and np.array_equal(s8, f["scale_fused"])
    assert np.array_equal(O.dequant_fp8(codes, scale), f["w_eff"])
    xf = O.bf16_bits_to_f32(f["x"])
    assert np.array_equal(O.gemv_ref(xf, f["w_eff"], O.EPI_SILU).astype(np.float32), f["out_plain_silu"])


# ---------------------------------------------------------------------------
# planted mistakes: the pins above must reject plausible wrong oracles
# ---------------------------------------------------------------------------


def test_planted_mistakes_are_caught():
    w, _, _ = O.synth(8, 256, 1, seed=18)
    q, s, lo, z = O.quantize_int4_asym(w, 128)
    sz = O.scales_zeros(s, z)
    good = O.dequant_int4_zp(q, sz, 128)

    # 1. zero point with the wrong sign of the 8-step offset
    bad = ((q.astype(np.float32) + 8) * np.repeat(O.round_bf16(s), 128, 1)
           + np.repeat(O.round_bf16(z), 128, 1))
    assert np.abs(bad - w).max() > 10 * np.abs(good - w).max()

    # 2. scales_zeros read as [N, G] instead of [G, N] (square case G == N)
    w2, _, _ = O.synth(2, 256, 1, seed=19)
    w2[0, 128:] *= 50.0                   # groups of very different scale
    q2, s2, _, z2 = O.quantize_int4_asym(w2, 128)
    sz2 = O.scales_zeros(s2, z2)
    bad2 = O.dequant_int4_zp(q2, np.swapaxes(sz2, 0, 1), 128)
    good2 = O.dequant_int4_zp(q2, sz2, 128)
    assert np.abs(bad2 - w2).max() > 3 * np.abs(good2 - w2).max()

    # 3. nibble order swapped: the single-nibble pin rejects it
    qq = np.zeros((1, 4), np.uint8)
    qq[0, 0] = 5
    assert O.pack_nibbles_odd_low(qq)[0, 0] != 5 and O.pack_nibbles_even_low(qq)[0, 0] == 5

    # 4. e4m3 decoded with exponent bias 8 instead of 7: torch's cast rejects it
    want = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    ok = ~np.isnan(want)
    assert not np.array_equal((O.e4m3fn_decode_table() / 2)[ok], want[ok])

    # 5. a GEMV that drops the residual fails the zero-W pin
    def gemv_no_res(x, w, epi=O.EPI_NONE, res=None):
        return np.asarray(x, np.float64) @ np.asarray(w, np.float64).T

    res = np.ones((1, 8))
    assert not np.array_equal(gemv_no_res(np.ones((1, 256)), np.zeros((8, 256)), O.EPI_RES, res), res)
    assert np.array_equal(O.gemv_ref(np.ones((1, 256)), np.zeros((8, 256)), O.EPI_RES, res), res)


# ---------------------------------------------------------------------------
# tiled layout (include/bz_gemv.h BZ_W_*_TILED[_PAIRED]): pinned against a
# scalar loop over its written definition, not the vectorised restatement
# ---------------------------------------------------------------------------


def _tile_scalar(rows_bytes, scales, int4, paired):
    """Byte-by-byte: logical row r -> block b, row t (paired: gate rows 8b+t,
    up rows 8b+t-8); unit u of the row at chunk(b) + 1024 u + 64 t; int4 (s, z)
    at chunk(b) + 1024 NU + 64 u + 4 t, fp8 row scale at chunk(b) + 1024 NU + 4 t."""
    n, rb = rows_bytes.shape
    nu = rb // 64
    chunk = (nu * 1024 + (nu * 64 if int4 else 64) + 127) // 128 * 128
    buf = bytearray((n // 16) * chunk)
    for r in range(n):
        if paired:
            h = n // 2
            b, t = ((r // 8, r % 8) if r < h else ((r - h) // 8, 8 + (r - h) % 8))
        else:
            b, t = r // 16, r % 16
        for u in range(nu):
            for i in range(64):
                buf[b * chunk + 1024 * u + 64 * t + i] = int(rows_bytes[r, 64 * u + i])
            if int4:
                for i in range(4):
                    buf[b * chunk + 1024 * nu + 64 * u + 4 * t + i] = int(scales[r, u, i])
        if not int4:
            for i in range(4):
                buf[b * chunk + 1024 * nu + 4 * t + i] = int(scales[r, i])
    return np.frombuffer(bytes(buf), dtype=np.uint8)


@pytest.mark.parametrize("paired", [False, True])
def test_tile_int4_matches_scalar_definition(paired):
    rng = np.random.default_rng(7)
    n, k = 32, 256
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    sz = rng.integers(0, 1 << 16, (k // 128, n, 2), dtype=np.uint16)
    got = O.tile_int4(packed, sz, paired)
    scales = np.ascontiguousarray(sz.transpose(1, 0, 2)).view(np.uint8).reshape(n, k // 128, 4)
    assert np.array_equal(got, _tile_scalar(packed, scales, True, paired))
    p2, s2 = O.untile_int4(got, n, k, paired)
    assert np.array_equal(p2, packed) and np.array_equal(s2, sz)


@pytest.mark.parametrize("paired", [False, True])
def test_tile_fp8_matches_scalar_definition(paired):
    rng = np.random.default_rng(8)
    n, k = 32, 192
    codes = rng.integers(0, 256, (n, k), dtype=np.uint8)
    scale = rng.standard_normal(n).astype(np.float32)
    got = O.tile_fp8(codes, scale, paired)
    assert np.array_equal(got, _tile_scalar(codes, scale.view(np.uint8).reshape(n, 4), False, paired))
    c2, s2 = O.untile_fp8(got, n, k, paired)
    assert np.array_equal(c2, codes) and np.array_equal(s2.view(np.uint32), scale.view(np.uint32))


def test_tile_paired_puts_gate_and_up_rows_in_one_block():
    """Block b of a paired [gate; up] weight holds gate rows 8b..8b+7 in tile
    rows 0-7 and up rows 8b..8b+7 in tile rows 8-15 (so it yields outputs
    8b..8b+7), and a chunk is a multiple of 128 bytes."""
    n, k = 64, 128
    rows = np.repeat(np.arange(n, dtype=np.uint8)[:, None], k // 2, axis=1)  # row r filled with byte r
    sz = np.zeros((1, n, 2), dtype=np.uint16)
    buf = O.tile_int4(rows, sz, paired=True)
    chunk = O.tiled_chunk_bytes(1, True)
    assert chunk % 128 == 0 and len(buf) == (n // 16) * chunk
    for b in range(n // 16):
        for t in range(16):
            want = 8 * b + t if t < 8 else n // 2 + 8 * b + t - 8
            assert buf[b * chunk + 64 * t] == want
