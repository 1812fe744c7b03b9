"""GPU parity of the tiled weight formats and the streaming GEMV that reads
them (path 5), through the C ABI, against the CPU oracle.

Bars:
  * packing, unpacking and indexing: bit-exact (device packer == the
    oracle's byte-by-byte restatement of the layout; dequantized tiled weights
    == dequantized row-major weights, bit for bit);
  * GEMV outputs: max|out-ref|/max|ref| <= 1e-2 (bench_gemv.py:53) against the
    float64 dequantize-then-matmul oracle on the same packed weights
    (bench_gemv.py:30-52), <= 4e-3 against the same-rounding oracle (a
    dropped term or a wrong row fails it), and within one bf16 step (2^-7 of
    the largest output) of the row-major GEMV of the same weights: both
    outputs are rounded to bf16, so they may differ by one step.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import bz_oracle as O
from tests._util import Fp8Case, Int4Case, bf16_bits, bf16_tensor, f32, u8_tensor

pytestmark = pytest.mark.gpu

TOL = 1e-2
TIGHT = 4e-3
ONE_BF16_STEP = 2.0 ** -7

from breeze_amd import gemv as G  # noqa: E402


def _rng(seed):
    return np.random.default_rng(seed)


def _int4_case(n, k, seed, symmetric=True):
    w = (_rng(seed).standard_normal((n, k)) * 0.02).astype(np.float32)
    return Int4Case(w, 128, symmetric=symmetric)


def _fp8_case(n, k, seed):
    w = (_rng(seed).standard_normal((n, k)) * 0.02).astype(np.float32)
    return Fp8Case(w)


def _tiled_i4(c, paired):
    fmt = G.W_INT4_TILED_PAIRED if paired else G.W_INT4_TILED
    return G.pack_tiled(G.W_INT4_ZP, c.d_packed, c.K, fmt, sc0=c.d_sz), fmt


def _tiled_f8(c, paired):
    fmt = G.W_FP8_TILED_PAIRED if paired else G.W_FP8_TILED
    return G.pack_tiled(G.W_FP8, c.d_codes, c.K, fmt, sc0=c.d_scale), fmt


# ---------------------------------------------------------------------------
# layout: bit-exact
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("paired", [False, True])
@pytest.mark.parametrize("n,k", [(16, 128), (48, 384), (64, 2560)])
def test_pack_int4_matches_oracle(paired, n, k):
    c = _int4_case(n, k, 1, symmetric=False)
    buf, _ = _tiled_i4(c, paired)
    want = O.tile_int4(c.packed, c.sz_bits, paired)
    assert np.array_equal(buf.cpu().numpy(), want)


@pytest.mark.parametrize("paired", [False, True])
@pytest.mark.parametrize("n,k", [(16, 64), (32, 192), (64, 2560)])
def test_pack_fp8_matches_oracle(paired, n, k):
    c = _fp8_case(n, k, 2)
    buf, _ = _tiled_f8(c, paired)
    want = O.tile_fp8(c.codes, c.scale, paired)
    assert np.array_equal(buf.cpu().numpy(), want)


def test_pack_halves_and_tiled_source():
    """[gate; up] packed by one call per half, and re-tiled from the plain
    tiled buffers of the halves, equals the one-call paired packing."""
    n, k = 64, 512
    c = _int4_case(n, k, 3)
    full = G.pack_tiled(G.W_INT4_ZP, c.d_packed, k, G.W_INT4_TILED_PAIRED, sc0=c.d_sz)
    h = n // 2
    gate_sz = bf16_tensor(np.ascontiguousarray(c.sz_bits[:, :h]))
    up_sz = bf16_tensor(np.ascontiguousarray(c.sz_bits[:, h:]))
    halves = torch.zeros_like(full)
    G.pack_tiled(G.W_INT4_ZP, c.d_packed[:h].contiguous(), k, G.W_INT4_TILED_PAIRED, sc0=gate_sz, n_total=n,
                 out=halves)
    G.pack_tiled(G.W_INT4_ZP, c.d_packed[h:].contiguous(), k, G.W_INT4_TILED_PAIRED, sc0=up_sz, n_total=n, row0=h,
                 out=halves)
    assert torch.equal(full, halves)
    g_t = G.pack_tiled(G.W_INT4_ZP, c.d_packed[:h].contiguous(), k, G.W_INT4_TILED, sc0=gate_sz)
    u_t = G.pack_tiled(G.W_INT4_ZP, c.d_packed[h:].contiguous(), k, G.W_INT4_TILED, sc0=up_sz)
    re = torch.zeros_like(full)
    G.pack_tiled(G.W_INT4_TILED, g_t, k, G.W_INT4_TILED_PAIRED, n_total=n, out=re)
    G.pack_tiled(G.W_INT4_TILED, u_t, k, G.W_INT4_TILED_PAIRED, n_total=n, row0=h, out=re)
    assert torch.equal(full, re)


@pytest.mark.parametrize("paired", [False, True])
def test_dequant_tiled_int4_equals_rowmajor(paired):
    c = _int4_case(96, 1024, 4, symmetric=False)
    buf, fmt = _tiled_i4(c, paired)
    got = f32(G.dequant(fmt, buf, c.N, c.K, group=128))
    want = f32(G.dequant(G.W_INT4_ZP, c.d_packed, c.N, c.K, sc0=c.d_sz, group=128))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(got.view(np.uint32), c.w_zp.view(np.uint32))


@pytest.mark.parametrize("paired", [False, True])
def test_dequant_tiled_fp8_equals_rowmajor(paired):
    c = _fp8_case(48, 640, 5)
    buf, fmt = _tiled_f8(c, paired)
    got = f32(G.dequant(fmt, buf, c.N, c.K))
    want = f32(G.dequant(G.W_FP8, c.d_codes, c.N, c.K, sc0=c.d_scale))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_single_nibble_sweep_tiled():
    """One non-zero nibble at every k of a row, through the tiled decoder:
    pins k -> (unit, lane piece, byte, nibble) of the tile."""
    K = 256
    q = np.zeros((K, K), dtype=np.uint8)
    q[np.arange(K), np.arange(K)] = np.arange(K) % 15 + 1
    packed = O.pack_nibbles_even_low(q)
    sz = O.scales_zeros(np.ones((K, K // 128), np.float32), np.zeros((K, K // 128), np.float32))
    buf = G.pack_tiled(G.W_INT4_ZP, u8_tensor(packed), K, G.W_INT4_TILED, sc0=bf16_tensor(sz))
    got = f32(G.dequant(G.W_INT4_TILED, buf, K, K, group=128))
    assert np.array_equal(got, q.astype(np.float32) - 8.0)


# ---------------------------------------------------------------------------
# GEMV: oracle and row-major path
# ---------------------------------------------------------------------------


def _x(m, k, seed):
    return O.f32_to_bf16_bits(_rng(seed).standard_normal((m, k)).astype(np.float32))


def _gamma(k, seed):
    return O.f32_to_bf16_bits((1 + 0.1 * _rng(seed).standard_normal(k)).astype(np.float32))


def _ref(x_bits, w_eff, gamma_bits, epi, res_bits):
    xf = O.bf16_bits_to_f32(x_bits)
    xn = O.rmsnorm_folded(xf, O.bf16_bits_to_f32(gamma_bits)) if gamma_bits is not None else xf
    res = O.bf16_bits_to_f32(res_bits) if res_bits is not None else None
    return O.gemv_ref(xn, w_eff, epi, res)


def _run_both(fmt_rm, rm_kw, fmt_t, tbuf, n, x_bits, gamma_bits, epi, res_bits):
    x = bf16_tensor(x_bits)
    gamma = bf16_tensor(gamma_bits) if gamma_bits is not None else None
    res = bf16_tensor(res_bits) if res_bits is not None else None
    out_t = G.gemv(x, tbuf, fmt_t, n, gamma=gamma, epilogue=epi, residual=res)
    out_r = G.gemv(x, rm_kw.pop("w"), fmt_rm, n, gamma=gamma, epilogue=epi, residual=res, **rm_kw)
    torch.cuda.synchronize()
    return f32(out_t), f32(out_r)


CASES_I4 = [
    # (n, k, norm, epilogue)
    (256, 1024, True, 1),
    (512, 2048, True, 0),
    (384, 1280, False, 2),
    (256, 4096, False, 2),
    (128, 10240, False, 2),
]


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 11])
@pytest.mark.parametrize("n,k,norm,epi", CASES_I4)
def test_gemv_tiled_int4(m, n, k, norm, epi):
    c = _int4_case(n, k, 10 + m)
    buf, fmt = _tiled_i4(c, epi == 1)
    x_bits = _x(m, k, 20 + m)
    gamma_bits = _gamma(k, 30) if norm else None
    n_out = n // 2 if epi == 1 else n
    res_bits = _x(m, n_out, 40) if epi == 2 else None
    got, rm = _run_both(G.W_INT4_ZP, {"w": c.d_packed, "sc0": c.d_sz, "group": 128}, fmt, buf, n, x_bits,
                        gamma_bits, epi, res_bits)
    ref = _ref(x_bits, c.w_zp, gamma_bits, epi, res_bits)
    assert O.rel_err(got, ref) <= TIGHT
    assert O.rel_err(got, rm) <= ONE_BF16_STEP


CASES_F8 = [
    (256, 1024, True, 1),
    (512, 2560, True, 0),
    (384, 1280, False, 2),
    (128, 10240, False, 2),
]


@pytest.mark.parametrize("m", [1, 2, 3, 4, 6, 8, 9])
@pytest.mark.parametrize("n,k,norm,epi", CASES_F8)
def test_gemv_tiled_fp8(m, n, k, norm, epi):
    c = _fp8_case(n, k, 50 + m)
    buf, fmt = _tiled_f8(c, epi == 1)
    x_bits = _x(m, k, 60 + m)
    gamma_bits = _gamma(k, 70) if norm else None
    n_out = n // 2 if epi == 1 else n
    res_bits = _x(m, n_out, 80) if epi == 2 else None
    got, rm = _run_both(G.W_FP8, {"w": c.d_codes, "sc0": c.d_scale}, fmt, buf, n, x_bits, gamma_bits, epi,
                        res_bits)
    ref = _ref(x_bits, c.w_eff, gamma_bits, epi, res_bits)
    assert O.rel_err(got, ref) <= TIGHT
    assert O.rel_err(got, rm) <= ONE_BF16_STEP


# RMSNorm over slices whose x and gamma loads exceed the kernel's register
# budget (rounds x (1 + rows) > 12: the later loads are issued during the
# staging).  Lanes past a wave's slice must read zeros there, or the row's
# sum of squares counts the slice's last block again (rows 2 and up of the
# launch then get a wrong 1/rms).  (fmt, n, k, epilogue, rows, cfg)
NORM_BEYOND_REGISTERS = [
    ("int4", 2048, 8192, 0, 5, (0, 0, 0, 0)),    # 13 waves x 5 units, 2 rounds
    ("int4", 2048, 8192, 0, 8, (0, 0, 0, 0)),
    ("int4", 1024, 10240, 1, 6, (0, 0, 0, 0)),   # paired, 16 waves x 5 units
    ("fp8", 2048, 10240, 0, 5, (0, 0, 0, 0)),    # 16 waves x 10 units, 2 rounds
    ("fp8", 2048, 10240, 2, 8, (0, 0, 0, 0)),
    ("int4", 512, 2560, 0, 6, (0, 4, 0, 5)),     # forced 4 waves x 5 units
    ("int4", 512, 2560, 0, 4, (0, 2, 0, 5)),     # forced 2 waves x 10 units, 3 rounds
    ("fp8", 512, 2560, 1, 6, (0, 4, 0, 5)),     # paired, forced 4 waves x 10 units
]


@pytest.mark.parametrize("fmt,n,k,epi,m,cfg", NORM_BEYOND_REGISTERS,
                         ids=[f"{c[0]}-n{c[1]}-k{c[2]}-e{c[3]}-m{c[4]}-w{c[5][1]}" for c in NORM_BEYOND_REGISTERS])
def test_gemv_tiled_norm_beyond_register_budget(fmt, n, k, epi, m, cfg):
    seed = 600 + m + k // 512
    c = _int4_case(n, k, seed) if fmt == "int4" else _fp8_case(n, k, seed)
    buf, tf = _tiled_i4(c, epi == 1) if fmt == "int4" else _tiled_f8(c, epi == 1)
    w_eff = c.w_zp if fmt == "int4" else c.w_eff
    x_bits = _x(m, k, seed + 1)
    # rows of very different scale, so a wrong 1/rms of any row shows
    x_bits = O.f32_to_bf16_bits(O.bf16_bits_to_f32(x_bits) * (1.0 + 3.0 * np.arange(m, dtype=np.float32))[:, None])
    gamma_bits = _gamma(k, seed + 2)
    n_out = n // 2 if epi == 1 else n
    res_bits = _x(m, n_out, seed + 3) if epi == 2 else None
    out = G.gemv(bf16_tensor(x_bits), buf, tf, n, gamma=bf16_tensor(gamma_bits), epilogue=epi,
                 residual=bf16_tensor(res_bits) if res_bits is not None else None, cfg=cfg)
    got = f32(out)
    ref = _ref(x_bits, w_eff, gamma_bits, epi, res_bits)
    for r in range(m):  # per row: a row with a wrong norm fails on its own
        assert O.rel_err(got[r:r + 1], ref[r:r + 1]) <= TIGHT, r


@pytest.mark.parametrize("waves", [1, 2, 3, 7, 16])
def test_gemv_tiled_forced_waves(waves):
    """Every wave count (uneven unit splits, idle waves) gives the same sums;
    one wave cannot hold the 20 units of a K = 2560 row (10 at most)."""
    n, k, m = 64, 2560, 2
    c = _int4_case(n, k, 90)
    buf, fmt = _tiled_i4(c, False)
    x = bf16_tensor(_x(m, k, 91))
    if waves == 1:
        with pytest.raises(RuntimeError, match="status 4"):
            G.gemv(x, buf, fmt, n, cfg=(0, waves, 0, 5))
        return
    got = f32(G.gemv(x, buf, fmt, n, cfg=(0, waves, 0, 5)))
    ref = _ref(_x(m, k, 91), c.w_zp, None, 0, None)
    assert O.rel_err(got, ref) <= TOL


def test_gemv_tiled_f32_out_and_residual():
    n, k, m = 128, 1024, 3
    c = _fp8_case(n, k, 93)
    buf, fmt = _tiled_f8(c, False)
    x_bits = _x(m, k, 94)
    res = torch.randn(m, n, device="cuda", dtype=torch.float32)
    out = G.gemv(bf16_tensor(x_bits), buf, fmt, n, epilogue=G.EPI_RESIDUAL, residual=res, out_dtype=torch.float32)
    ref = O.gemv_ref(O.bf16_bits_to_f32(x_bits), c.w_eff, O.EPI_RES, res.cpu().numpy())
    assert out.dtype == torch.float32
    assert O.rel_err(f32(out), ref) <= TOL


@pytest.mark.parametrize(
    "fmt,n,k,m",
    [
        ("int4", 2048, 6144, 3), ("int4", 2048, 6144, 7), ("int4", 1024, 8192, 8),
        ("fp8", 1024, 8192, 5), ("fp8", 2560, 4096, 7), ("fp8", 1536, 1024, 6),
    ],
)
def test_gemv_several_rows_streaming_residual_f32(fmt, n, k, m):
    """Several rows over K <= 8192 on the automatic path (the several-block
    kernel in one launch, ragged row counts included) with an fp32 residual
    and fp32 output, against the oracle; the same call with a bf16 residual
    and output agrees to the bf16 bar."""
    c = _int4_case(n, k, 760 + m) if fmt == "int4" else _fp8_case(n, k, 761 + m)
    buf, tf = _tiled_i4(c, False) if fmt == "int4" else _tiled_f8(c, False)
    w_eff = c.w_zp if fmt == "int4" else c.w_eff
    x_bits = _x(m, k, 762 + m)
    res = torch.randn(m, n, device="cuda", dtype=torch.float32)
    out = G.gemv(bf16_tensor(x_bits), buf, tf, n, epilogue=G.EPI_RESIDUAL, residual=res, out_dtype=torch.float32)
    assert out.dtype == torch.float32
    ref = O.gemv_ref(O.bf16_bits_to_f32(x_bits), w_eff, O.EPI_RES, res.cpu().numpy())
    assert O.rel_err(f32(out), ref) <= TOL
    res16 = res.to(torch.bfloat16)
    out16 = G.gemv(bf16_tensor(x_bits), buf, tf, n, epilogue=G.EPI_RESIDUAL, residual=res16)
    ref16 = O.gemv_ref(O.bf16_bits_to_f32(x_bits), w_eff, O.EPI_RES, res16.float().cpu().numpy())
    assert O.rel_err(f32(out16), ref16) <= TIGHT


def test_gemv_tiled_rejects_wrong_epilogue_and_size():
    n, k = 64, 256
    c = _int4_case(n, k, 95)
    plain, _ = _tiled_i4(c, False)
    paired, _ = _tiled_i4(c, True)
    x = bf16_tensor(_x(1, k, 96))
    with pytest.raises(RuntimeError):
        G.gemv(x, plain, G.W_INT4_TILED, n, epilogue=G.EPI_SILU_GATE)
    with pytest.raises(RuntimeError):
        G.gemv(x, paired, G.W_INT4_TILED_PAIRED, n)
    with pytest.raises(ValueError):
        G.gemv(x, plain[:-128], G.W_INT4_TILED, n)


# ---------------------------------------------------------------------------
# the benchmark configurations' shapes at full size
# ---------------------------------------------------------------------------

FULL = [
    # (name, fmt, n, k, norm, epilogue)
    ("C2 gate|up", "int4", 20480, 2560, True, 1),
    ("C2 down", "int4", 2560, 10240, False, 2),
    ("C3 qkv", "fp8", 4096, 2560, True, 0),
    ("C3 o_proj", "fp8", 2560, 4096, False, 2),
    ("C3 gate|up", "fp8", 20480, 2560, True, 1),
    ("C3 down", "fp8", 2560, 10240, False, 2),
    ("C5 qkv", "int4", 6144, 2560, True, 0),
    ("C5 o_proj", "int4", 2560, 4096, False, 2),
]


_FULL_CACHE: dict = {}


def _full_case(name, fmt, n, k, epi, seed):
    if name not in _FULL_CACHE:
        _FULL_CACHE.clear()  # one full-size weight at a time
        if fmt == "int4":
            c = _int4_case(n, k, seed)
            buf, tf = _tiled_i4(c, epi == 1)
            _FULL_CACHE[name] = (buf, tf, c.w_zp)
        else:
            c = _fp8_case(n, k, seed)
            buf, tf = _tiled_f8(c, epi == 1)
            _FULL_CACHE[name] = (buf, tf, c.w_eff)
    return _FULL_CACHE[name]


@pytest.mark.parametrize("name,fmt,n,k,norm,epi", FULL, ids=[f[0] for f in FULL])
@pytest.mark.parametrize("m", [1, 2])
def test_gemv_tiled_full_size(name, fmt, n, k, norm, epi, m):
    seed = sum(name.encode()) % 1000
    buf, tf, w_eff = _full_case(name, fmt, n, k, epi, seed)
    x_bits = _x(m, k, seed + 1)
    gamma_bits = _gamma(k, seed + 2) if norm else None
    n_out = n // 2 if epi == 1 else n
    res_bits = _x(m, n_out, seed + 3) if epi == 2 else None
    out = G.gemv(bf16_tensor(x_bits), buf, tf, n, gamma=bf16_tensor(gamma_bits) if norm else None, epilogue=epi,
                 residual=bf16_tensor(res_bits) if res_bits is not None else None)
    ref = _ref(x_bits, w_eff, gamma_bits, epi, res_bits)
    assert O.rel_err(f32(out), ref) <= TOL


def test_gemv_tiled_graph_replays_bit_identical():
    n, k, m = 2048, 2560, 2
    c = _int4_case(n, k, 97)
    buf, fmt = _tiled_i4(c, True)
    x = bf16_tensor(_x(m, k, 98))
    gamma = bf16_tensor(_gamma(k, 99))
    out = torch.empty(m, n // 2, device="cuda", dtype=torch.bfloat16)
    G.gemv(x, buf, fmt, n, gamma=gamma, epilogue=G.EPI_SILU_GATE, out=out)
    torch.cuda.synchronize()
    eager = out.clone()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st), torch.cuda.graph(g, stream=st):
        G.gemv(x, buf, fmt, n, gamma=gamma, epilogue=G.EPI_SILU_GATE, out=out)
    torch.cuda.current_stream().wait_stream(st)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


@pytest.mark.parametrize("m", [1, 2, 3, 9])
def test_gemv_tiled_second_store(m):
    """out2 receives columns [0, n2) of the same launch's result bit for bit
    (the query part of a QKV projection handed to the next kernel), at M
    spanning two launches (9 = 8 + 1 rows), and leaves the rest of out2's
    rows untouched."""
    n, k, n2 = 6144, 2560, 4096
    c = _int4_case(n, k, 900 + m)
    tbuf, fmt = _tiled_i4(c, False)
    x, g = _x(m, k, 901 + m), _gamma(k, 902 + m)
    out = G.gemv(bf16_tensor(x), tbuf, fmt, n, gamma=bf16_tensor(g))
    wide = torch.full((m, n2 + 24), -7.0, device="cuda", dtype=torch.bfloat16)
    out2 = wide[:, 8: 8 + n2]
    got = G.gemv(bf16_tensor(x), tbuf, fmt, n, gamma=bf16_tensor(g), out2=out2)
    assert torch.equal(got, out)
    assert torch.equal(out2, out[:, :n2])
    assert bool((wide[:, :8] == -7).all()) and bool((wide[:, 8 + n2:] == -7).all())
    ref = _ref(x, c.w_zp, g, O.EPI_NONE, None)
    assert O.rel_err(f32(got), ref) <= TIGHT


def test_gemv_tiled_second_store_paired_f32():
    """The second store on a paired SiLU-gate GEMV with fp32 output and a
    column count that is not a multiple of a row block (100 of 256)."""
    n, k, m, n2 = 512, 1024, 2, 100
    c = _fp8_case(n, k, 910)
    tbuf, fmt = _tiled_f8(c, True)
    x = _x(m, k, 911)
    out = G.gemv(bf16_tensor(x), tbuf, fmt, n, epilogue=G.EPI_SILU_GATE, out_dtype=torch.float32)
    out2 = torch.zeros(m, n2, device="cuda", dtype=torch.float32)
    got = G.gemv(bf16_tensor(x), tbuf, fmt, n, epilogue=G.EPI_SILU_GATE, out_dtype=torch.float32, out2=out2)
    assert torch.equal(got, out) and torch.equal(out2, out[:, :n2])
    with pytest.raises(ValueError, match="out2"):
        G.gemv(bf16_tensor(x), tbuf, fmt, n, epilogue=G.EPI_SILU_GATE, out2=torch.zeros(m, n2, device="cuda"))


# ---------------------------------------------------------------------------
# several rows: the tile kernel over the tiled formats
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("fmt", ["int4", "fp8"])
@pytest.mark.parametrize("m", [5, 8, 9, 16, 17, 32, 40])
def test_tile_kernel_reads_tiled_formats(fmt, m):
    """The several-row tile kernel (path 4) reads a tiled weight in place: the
    result is bit-identical to the same kernel over the row-major weight
    (same launch plan, same arithmetic) and within the bar of the oracle.
    The automatic choice for this shape is the several-block streaming kernel
    with one block per workgroup up to 8 rows (one launch) and the panel
    kernel (path 6) beyond."""
    n, k = 2560, 2560
    c = _int4_case(n, k, 950 + m) if fmt == "int4" else _fp8_case(n, k, 960 + m)
    tbuf, tf = _tiled_i4(c, False) if fmt == "int4" else _tiled_f8(c, False)
    x = _x(m, k, 970 + m)
    res = _x(m, n, 980 + m)
    got = G.gemv(bf16_tensor(x), tbuf, tf, n, epilogue=G.EPI_RESIDUAL, residual=bf16_tensor(res), cfg=(0, 0, 0, 4))
    if fmt == "int4":
        want = G.gemv(bf16_tensor(x), c.d_packed, G.W_INT4_ZP, n, sc0=c.d_sz, epilogue=G.EPI_RESIDUAL,
                      residual=bf16_tensor(res), cfg=(0, 0, 0, 4))
        w_eff = c.w_zp
    else:
        want = G.gemv(bf16_tensor(x), c.d_codes, G.W_FP8, n, sc0=c.d_scale, epilogue=G.EPI_RESIDUAL,
                      residual=bf16_tensor(res), cfg=(0, 0, 0, 4))
        w_eff = c.w_eff
    assert torch.equal(got, want)
    auto = G.gemv(bf16_tensor(x), tbuf, tf, n, epilogue=G.EPI_RESIDUAL, residual=bf16_tensor(res))
    panel = G.gemv(bf16_tensor(x), tbuf, tf, n, epilogue=G.EPI_RESIDUAL, residual=bf16_tensor(res),
                   cfg=(0, 0, 0, 6))
    wide = G.gemv(bf16_tensor(x), tbuf, tf, n, epilogue=G.EPI_RESIDUAL, residual=bf16_tensor(res),
                  cfg=(0, 0, 1, 5))
    assert torch.equal(auto, wide if m <= 8 else panel)
    assert O.rel_err(f32(panel), _ref(x, w_eff, None, O.EPI_RES, res)) <= TIGHT
    assert O.rel_err(f32(wide), _ref(x, w_eff, None, O.EPI_RES, res)) <= TIGHT
    assert O.rel_err(f32(got), _ref(x, w_eff, None, O.EPI_RES, res)) <= TIGHT


@pytest.mark.parametrize("slices", [4, 5, 8])
def test_tile_kernel_tiled_forced_slices(slices):
    """Forced K slices (split-K partials and the last arrival's sum) over a
    tiled int4 weight, K10240 N2560 (down) at M = 16, against the row-major
    weight through the same plan."""
    n, k, m = 2560, 10240, 16
    c = _int4_case(n, k, 990)
    tbuf, tf = _tiled_i4(c, False)
    x = bf16_tensor(_x(m, k, 991))
    cfg = (0, 0, 0, 4, slices)
    got = G.gemv(x, tbuf, tf, n, cfg=cfg)
    want = G.gemv(x, c.d_packed, G.W_INT4_ZP, n, sc0=c.d_sz, cfg=cfg)
    assert torch.equal(got, want)
    assert O.rel_err(f32(got), _ref(_x(m, k, 991), c.w_zp, None, O.EPI_NONE, None)) <= TIGHT


def test_tile_kernel_not_taken_with_norm_silu_or_second_store():
    """RMSNorm, SiLU-gate and the second store stay on the streaming kernel
    at any M (the tile kernel has none of them); forcing path 4 for a paired
    weight is refused."""
    n, k, m = 512, 1024, 12
    c = _int4_case(n, k, 995)
    tp, tfp = _tiled_i4(c, True)
    x, g = _x(m, k, 996), _gamma(k, 997)
    out = G.gemv(bf16_tensor(x), tp, tfp, n, gamma=bf16_tensor(g), epilogue=G.EPI_SILU_GATE)
    assert O.rel_err(f32(out), _ref(x, c.w_zp, g, O.EPI_SILU, None)) <= TIGHT
    with pytest.raises(RuntimeError, match="status 4"):
        G.gemv(bf16_tensor(x), tp, tfp, n, gamma=bf16_tensor(g), epilogue=G.EPI_SILU_GATE, cfg=(0, 0, 0, 4))
    t, tf = _tiled_i4(c, False)
    out2 = torch.zeros(m, 64, device="cuda", dtype=torch.bfloat16)
    out = G.gemv(bf16_tensor(x), t, tf, n, out2=out2)
    assert torch.equal(out2, out[:, :64])


def test_stream_read_writes_only_on_key_match():
    """The read-floor kernel reads every chunk and writes its sink only when a
    thread's XOR equals the key: zeros with key 1 leave the sink alone, key 0
    writes 0; an empty launch writes nothing."""
    buf = torch.zeros(850 * 16384 // 4, dtype=torch.int32, device="cuda")
    sink = torch.full((4,), 7, dtype=torch.int32, device="cuda")
    G.stream_read(buf, sink, chunk=16384, key=1)
    G.stream_read(buf, sink, chunk=16384 * 5, key=1)
    G.stream_read(None, sink)
    torch.cuda.synchronize()
    assert sink.tolist() == [7, 7, 7, 7]
    G.stream_read(buf, sink, chunk=16384 * 10, key=0)
    torch.cuda.synchronize()
    assert sink.tolist() == [0, 7, 7, 7]


def test_shared_read_reads_x_and_own_chunk():
    """The whole-K read floor: every workgroup reads all of x (40960 bytes,
    not a whole number of its rounds) and workgroup b reads w's chunk b: a
    word planted near the end of x and one in workgroup 3's chunk each reach
    a thread's XOR."""
    x = torch.zeros(40960 // 4, dtype=torch.int32, device="cuda")
    w = torch.zeros(4 * 8192 // 4, dtype=torch.int32, device="cuda")
    x[(40960 - 16 * 7) // 4] = 0x1234
    w[(3 * 8192 + 9 * 16 + 8) // 4] = 0x777      # workgroup 3
    sink = torch.full((4,), 7, dtype=torch.int32, device="cuda")
    G.shared_read(x, w, 8192, 4, sink, key=0x999)
    torch.cuda.synchronize()
    assert sink.tolist() == [7, 7, 7, 7]
    for key in (0x1234, 0x777, 0):
        sink.fill_(7)
        G.shared_read(x, w, 8192, 4, sink, key=key)
        torch.cuda.synchronize()
        assert sink.tolist() == [key, 7, 7, 7]
    with pytest.raises(ValueError):
        G.shared_read(x, w, 8192, 5, sink)      # w shorter than 5 chunks


# ---------------------------------------------------------------------------
# the several-block streaming kernel (path 5 with cfg_tiles = blocks per
# workgroup; the rule's choice for weights of more than 256 row blocks)
# ---------------------------------------------------------------------------

WIDE = [
    # (fmt, n, k, norm, epilogue, blocks per workgroup)
    ("int4", 2048, 2560, True, 1, 5),     # paired, 128 blocks / 5: a ragged last workgroup (3 blocks)
    ("int4", 1536, 1024, False, 2, 3),
    ("int4", 768, 4096, True, 0, 8),      # 48 blocks / 8
    ("int4", 512, 10240, False, 0, 2),    # 80 units: 16 waves x 5
    ("fp8", 2048, 2560, True, 1, 5),
    ("fp8", 1024, 10240, False, 2, 1),    # one block per workgroup, all tiles in flight
    ("fp8", 1280, 1024, True, 0, 7),
]


@pytest.mark.parametrize("m", [1, 2, 3, 5, 8, 9])
@pytest.mark.parametrize("fmt,n,k,norm,epi,T", WIDE, ids=[f"{w[0]}-n{w[1]}-k{w[2]}-e{w[4]}-T{w[5]}" for w in WIDE])
def test_gemv_wide_matches_oracle_and_one_block_kernel(fmt, n, k, norm, epi, T, m):
    seed = 700 + T + m + k // 1024
    c = _int4_case(n, k, seed) if fmt == "int4" else _fp8_case(n, k, seed)
    buf, tf = _tiled_i4(c, epi == 1) if fmt == "int4" else _tiled_f8(c, epi == 1)
    w_eff = c.w_zp if fmt == "int4" else c.w_eff
    x_bits = _x(m, k, seed + 1)
    gamma_bits = _gamma(k, seed + 2) if norm else None
    n_out = n // 2 if epi == 1 else n
    res_bits = _x(m, n_out, seed + 3) if epi == 2 else None
    kw = dict(gamma=bf16_tensor(gamma_bits) if norm else None, epilogue=epi,
              residual=bf16_tensor(res_bits) if res_bits is not None else None)
    wide = G.gemv(bf16_tensor(x_bits), buf, tf, n, cfg=(0, 0, T, 5), **kw)
    one = G.gemv(bf16_tensor(x_bits), buf, tf, n, cfg=(0, 0, 0, 5), **kw)
    ref = _ref(x_bits, w_eff, gamma_bits, epi, res_bits)
    assert O.rel_err(f32(wide), ref) <= TIGHT
    # the same sums in another order (the waves' partials added in wave order
    # rather than by a DPP tree): within one bf16 step of the one-block kernel
    assert O.rel_err(f32(wide), f32(one)) <= ONE_BF16_STEP
    # deterministic: a second call is bit-identical
    assert torch.equal(G.gemv(bf16_tensor(x_bits), buf, tf, n, cfg=(0, 0, T, 5), **kw), wide)


@pytest.mark.parametrize("waves", [4, 5, 7, 16])
def test_gemv_wide_forced_waves_and_second_store(waves):
    """Forced wave counts (uneven unit splits) and the second store on the
    several-block kernel: out2 gets columns [0, n2) of the same launch."""
    n, k, m, n2, T = 6144, 2560, 3, 4096, 2
    c = _int4_case(n, k, 720 + waves)
    buf, tf = _tiled_i4(c, False)
    x, g = _x(m, k, 721), _gamma(k, 722)
    out2 = torch.zeros(m, n2, device="cuda", dtype=torch.bfloat16)
    got = G.gemv(bf16_tensor(x), buf, tf, n, gamma=bf16_tensor(g), out2=out2, cfg=(0, waves, T, 5))
    assert torch.equal(out2, got[:, :n2])
    assert O.rel_err(f32(got), _ref(x, c.w_zp, g, O.EPI_NONE, None)) <= TIGHT


def test_gemv_wide_rule_at_full_size():
    """The rule's automatic choice for the gate|up K2560 N20480 and the qkv
    K2560 N6144 (more than 256 row blocks) and for fp8 rows of K >= 4096 is
    the several-block kernel: the automatic result equals the one forced with
    the rule's block count bit for bit."""
    for fmt, n, k, epi, T in (("int4", 20480, 2560, 1, 5), ("fp8", 20480, 2560, 1, 5), ("int4", 6144, 2560, 0, 2),
                              ("fp8", 2560, 4096, 0, 1), ("fp8", 2560, 10240, 0, 1)):
        c = _int4_case(n, k, 730) if fmt == "int4" else _fp8_case(n, k, 731)
        buf, tf = _tiled_i4(c, epi == 1) if fmt == "int4" else _tiled_f8(c, epi == 1)
        x, g = _x(2, k, 732), _gamma(k, 733)
        auto = G.gemv(bf16_tensor(x), buf, tf, n, gamma=bf16_tensor(g), epilogue=epi)
        forced = G.gemv(bf16_tensor(x), buf, tf, n, gamma=bf16_tensor(g), epilogue=epi, cfg=(0, 0, T, 5))
        assert torch.equal(auto, forced), (fmt, n)
        w_eff = c.w_zp if fmt == "int4" else c.w_eff
        assert O.rel_err(f32(auto), _ref(x, w_eff, g, epi, None)) <= TIGHT


@pytest.mark.parametrize(
    "fmt,n,k,m,T",
    [
        ("int4", 2560, 4096, 3, 1),    # one block per workgroup from 3 rows over K <= 8192
        ("fp8", 4096, 2560, 4, 1),
        ("int4", 2560, 4096, 5, 1),    # 5-8 rows: one streaming launch, not the panel kernel
        ("fp8", 4096, 2560, 8, 1),
        ("fp8", 2048, 2048, 6, 1),
        ("int4", 6144, 2560, 7, 2),    # more than 256 blocks: the block count of the rule
        ("fp8", 20480, 2560, 3, 5),    # no longer the panel kernel at 3-4 rows
        ("int4", 20480, 2560, 8, 5),
        ("int4", 2048, 6144, 4, 1),    # K up to 8192
        ("int4", 2048, 6144, 8, 1),
        ("fp8", 1024, 8192, 6, 1),
    ],
)
def test_gemv_wide_rule_several_rows(fmt, n, k, m, T):
    """From 3 to 8 rows over rows of K <= 8192 (unpaired, no RMSNorm) the
    built-in rule runs the several-block kernel in one launch: the automatic
    result equals the one forced with the rule's block count bit for bit."""
    from breeze_amd import tuning

    saved = dict(tuning._TABLES)
    tuning._TABLES.clear()
    tuning._TABLES[tuning.arch_of(torch.device("cuda"))] = {}  # the built-in rule, not the table
    try:
        c = _int4_case(n, k, 750) if fmt == "int4" else _fp8_case(n, k, 751)
        buf, tf = _tiled_i4(c, False) if fmt == "int4" else _tiled_f8(c, False)
        x = _x(m, k, 752)
        auto = G.gemv(bf16_tensor(x), buf, tf, n)
        forced = G.gemv(bf16_tensor(x), buf, tf, n, cfg=(0, 0, T, 5))
        assert torch.equal(auto, forced), (fmt, n, k, m)
        w_eff = c.w_zp if fmt == "int4" else c.w_eff
        assert O.rel_err(f32(auto), _ref(x, w_eff, None, 0, None)) <= TIGHT
    finally:
        tuning._TABLES.clear()
        tuning._TABLES.update(saved)


def test_gemv_wide_rejects_bad_block_counts():
    n, k = 256, 1024
    c = _int4_case(n, k, 740)
    buf, tf = _tiled_i4(c, False)
    x = bf16_tensor(_x(1, k, 741))
    with pytest.raises(RuntimeError, match="status 1"):
        G.gemv(x, buf, tf, n, cfg=(0, 0, 9, 5))
