"""GPU parity of the several-row panel kernel (GEMV path 6: up to 32 rows of x
against an unpaired tiled int4 / fp8 weight, every workgroup covering the
whole K of its row blocks or one of several K slices, x read straight into
the matrix-core operands) through the C ABI, against the CPU oracle.

Bars as for the other GEMV paths:
  * max|out-ref|/max|ref| <= 4e-3 against the float64 dequantize-then-matmul
    of the same packed weights (bench_gemv.py:30-53; the reference's bar is
    1e-2), asymmetric int4 (z != 0) included;
  * one-hot rows of x with dyadic scales are bit-exact: every k of every unit
    lands on its own weight (pins the cross-lane redistribution of the tile
    pieces, the x piece offsets, the nibble order and the (s, z) rows);
  * repeated calls and graph replays are bit-identical (fixed summation
    order over the waves).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import bz_oracle as O
from tests._util import Fp8Case, Int4Case, bf16_tensor, f32, u8_tensor

pytestmark = pytest.mark.gpu

TOL = 1e-2
TIGHT = 4e-3
PANEL = 6

from breeze_amd import gemv as G  # noqa: E402


def _rng(seed):
    return np.random.default_rng(seed)


def _x(m, k, seed):
    return O.f32_to_bf16_bits(_rng(seed).standard_normal((m, k)).astype(np.float32))


def _weight(fmt, n, k, seed, symmetric=False):
    """(tiled buffer, format, W_eff) of an oracle-quantized N(0, 0.02) weight."""
    w = (_rng(seed).standard_normal((n, k)) * 0.02).astype(np.float32)
    if fmt == "int4":
        c = Int4Case(w, 128, symmetric=symmetric)
        return G.pack_tiled(G.W_INT4_ZP, c.d_packed, k, G.W_INT4_TILED, sc0=c.d_sz), G.W_INT4_TILED, c.w_zp
    c = Fp8Case(w)
    return G.pack_tiled(G.W_FP8, c.d_codes, k, G.W_FP8_TILED, sc0=c.d_scale), G.W_FP8_TILED, c.w_eff


def _run(buf, wf, n, x_bits, cfg=(0, 0, 0, PANEL), res_bits=None, out_dtype=torch.bfloat16):
    epi = G.EPI_RESIDUAL if res_bits is not None else G.EPI_NONE
    return G.gemv(bf16_tensor(x_bits), buf, wf, n, epilogue=epi, cfg=cfg, out_dtype=out_dtype,
                  residual=bf16_tensor(res_bits) if res_bits is not None else None)


def _ref(x_bits, w_eff, res_bits=None):
    res = O.bf16_bits_to_f32(res_bits) if res_bits is not None else None
    return O.gemv_ref(O.bf16_bits_to_f32(x_bits), w_eff, O.EPI_RES if res is not None else O.EPI_NONE, res)


# Shapes: 3 blocks, 7 blocks (a partial last workgroup for 2-5 blocks per
# workgroup), 160 blocks; K = 3 / 10 / 20 int4 units (6 / 20 / 40 fp8 units).
SHAPES = [(48, 384), (112, 1280), (2560, 2560)]


@pytest.mark.parametrize("fmt", ["int4", "fp8"])
@pytest.mark.parametrize("n,k", SHAPES)
@pytest.mark.parametrize("m", [1, 3, 16, 17, 32, 40])
@pytest.mark.parametrize("blocks", [1, 3, 5])
def test_panel_matches_oracle(fmt, n, k, m, blocks):
    buf, wf, w_eff = _weight(fmt, n, k, n + k + m, symmetric=(m % 2 == 0))
    x = _x(m, k, 7 * m + blocks)
    res = _x(m, n, 11 * m + blocks) if blocks != 3 else None
    got = _run(buf, wf, n, x, cfg=(0, 0, blocks, PANEL), res_bits=res,
               out_dtype=torch.float32 if m == 17 else torch.bfloat16)
    assert O.rel_err(f32(got), _ref(x, w_eff, res)) <= TIGHT


@pytest.mark.parametrize("fmt", ["int4", "fp8"])
@pytest.mark.parametrize("waves,blocks", [(1, 1), (3, 1), (7, 1), (16, 1), (1, 2), (5, 4), (8, 5)])
def test_panel_forced_waves(fmt, waves, blocks):
    """Every unit split (a last wave with fewer units reads zeros past the
    row) gives the oracle's result."""
    n, k, m = 224, 2560, 24
    buf, wf, w_eff = _weight(fmt, n, k, 300 + waves)
    x = _x(m, k, 301)
    units = k // (128 if fmt == "int4" else 64)
    if -(-units // waves) > 10:  # more units per wave than the kernel is built for
        with pytest.raises(RuntimeError, match="status 4"):
            _run(buf, wf, n, x, cfg=(0, waves, blocks, PANEL))
        return
    got = _run(buf, wf, n, x, cfg=(0, waves, blocks, PANEL))
    assert O.rel_err(f32(got), _ref(x, w_eff)) <= TIGHT


def _one_hot_rows(K, m_rows, shift):
    x = np.zeros((m_rows, K), dtype=np.float32)
    ks = (np.arange(m_rows) * 37 + shift) % K
    x[np.arange(m_rows), ks] = 1.0
    return O.f32_to_bf16_bits(x), ks


def test_panel_one_hot_int4_bit_exact():
    """x row m = e_{k_m}: out[m][n] = (q - 8) s + z of weight n at k_m,
    exactly (dyadic s and z, integer q), for k_m over every k of every unit."""
    N, K = 48, 512
    r = _rng(41)
    q = r.integers(0, 16, size=(N, K), dtype=np.uint8)
    s = (2.0 ** r.integers(-6, -2, size=(N, K // 128))).astype(np.float32)
    z = (r.integers(-8, 9, size=(N, K // 128)) * 2.0 ** -5).astype(np.float32)
    sz = O.scales_zeros(s, z)
    buf = G.pack_tiled(G.W_INT4_ZP, u8_tensor(O.pack_nibbles_even_low(q)), K, G.W_INT4_TILED, sc0=bf16_tensor(sz))
    w_eff = O.dequant_int4_zp(q, sz, 128)
    seen = set()
    for shift in range(16):
        x, ks = _one_hot_rows(K, 32, shift * 32)
        got = f32(_run(buf, G.W_INT4_TILED, N, x, out_dtype=torch.float32))
        assert np.array_equal(got, w_eff[:, ks].T), shift
        seen.update(ks.tolist())
    assert len(seen) == K


def test_panel_one_hot_fp8_bit_exact():
    N, K = 48, 512
    r = _rng(42)
    codes = r.integers(0, 256, size=(N, K), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x3C  # no NaN codes
    scale = (2.0 ** r.integers(-4, 2, size=N)).astype(np.float32)
    buf = G.pack_tiled(G.W_FP8, u8_tensor(codes), K, G.W_FP8_TILED, sc0=torch.from_numpy(scale).cuda())
    w_eff = O.dequant_fp8(codes, scale)
    seen = set()
    for shift in range(16):
        x, ks = _one_hot_rows(K, 32, shift * 32)
        got = f32(_run(buf, G.W_FP8_TILED, N, x, out_dtype=torch.float32))
        assert np.array_equal(got, w_eff[:, ks].T), shift
        seen.update(ks.tolist())
    assert len(seen) == K


# The several-row configuration's shapes (MTP draft verification + CFG).
FULL = [("int4", 20480, 2560), ("fp8", 20480, 2560), ("int4", 2560, 10240), ("fp8", 2560, 10240),
        ("int4", 10240, 2560), ("int4", 6144, 2560)]


@pytest.mark.parametrize("fmt,n,k", FULL, ids=[f"{f}-N{n}-K{k}" for f, n, k in FULL])
@pytest.mark.parametrize("m", [3, 8, 32])
def test_panel_full_size(fmt, n, k, m):
    buf, wf, w_eff = _weight(fmt, n, k, 500 + m, symmetric=True)
    x = _x(m, k, 501 + m)
    a = _run(buf, wf, n, x)
    b = _run(buf, wf, n, x)
    assert torch.equal(a, b)
    e = O.rel_err(f32(a), _ref(x, w_eff))
    assert e <= TIGHT, e


def test_panel_automatic_choice():
    """The built-in rule takes the panel kernel from 5 rows on, except 5-8
    rows over K <= 8192, which the several-block streaming kernel runs in one
    launch; at 3 rows the streaming kernel too.  Each automatic result is
    bit-identical to the one forced with the expected launch (a comparison
    against the other path would not tell them apart: after rounding to
    bf16 their sums in another order agree on most inputs)."""
    from breeze_amd import tuning

    wide = lambda t: (0, 0, t, 5)  # noqa: E731
    saved = dict(tuning._TABLES)
    tuning._TABLES.clear()
    tuning._TABLES[tuning.arch_of(torch.device("cuda"))] = {}  # the built-in rule, not the table
    try:
        for fmt, n, k, m, cfg in [("int4", 2560, 10240, 16, (0, 0, 0, PANEL)), ("int4", 2560, 4096, 32, (0, 0, 0, PANEL)),
                                  ("fp8", 20480, 2560, 3, wide(5)), ("int4", 2560, 10240, 32, (0, 0, 0, PANEL)),
                                  ("fp8", 2560, 10240, 32, (0, 0, 0, PANEL)), ("int4", 20480, 2560, 3, wide(5)),
                                  ("int4", 2560, 4096, 8, wide(1)), ("fp8", 4096, 2560, 5, wide(1)),
                                  ("fp8", 2560, 10240, 8, (0, 0, 0, PANEL)), ("int4", 2048, 2048, 12, (0, 0, 0, PANEL)),
                                  ("fp8", 1024, 8192, 8, wide(1)), ("int4", 2048, 6144, 6, wide(1))]:
            buf, wf, w_eff = _weight(fmt, n, k, 600 + m)
            x = _x(m, k, 601)
            auto = _run(buf, wf, n, x, cfg=(0, 0, 0, 0))
            forced = _run(buf, wf, n, x, cfg=cfg)
            assert torch.equal(auto, forced), (fmt, n, k, m, cfg)
            assert O.rel_err(f32(auto), _ref(x, w_eff)) <= TIGHT
    finally:
        tuning._TABLES.clear()
        tuning._TABLES.update(saved)


def test_panel_graph_replays_match_eager():
    n, k, m = 1280, 2560, 20
    buf, wf, _ = _weight("int4", n, k, 700)
    x = bf16_tensor(_x(m, k, 701))
    res = bf16_tensor(_x(m, n, 702))
    out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    call = lambda: G.gemv(x, buf, wf, n, epilogue=G.EPI_RESIDUAL, residual=res, out=out, cfg=(0, 0, 0, PANEL))
    call()
    torch.cuda.synchronize()
    want = out.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side), torch.cuda.graph(g, stream=side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    for i in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), i
        _ = (x.float() * 2).sum().item()  # eager work between replays


@pytest.mark.parametrize("fmt", ["int4", "fp8"])
def test_panel_fp32_residual_aliasing_out(fmt):
    n, k, m = 320, 1280, 12
    buf, wf, w_eff = _weight(fmt, n, k, 800)
    x = _x(m, k, 801)
    r = _rng(802).standard_normal((m, n)).astype(np.float32)
    out = torch.from_numpy(r.copy()).cuda()
    G.gemv(bf16_tensor(x), buf, wf, n, epilogue=G.EPI_RESIDUAL, residual=out, out=out, cfg=(0, 0, 0, PANEL))
    ref = O.gemv_ref(O.bf16_bits_to_f32(x), w_eff, O.EPI_RES, r)
    assert O.rel_err(f32(out), ref) <= TIGHT


def test_panel_rejects_what_it_cannot_run():
    """Path 6 takes unpaired tiled weights without RMSNorm or the second
    store, 1-5 blocks and at most 16 waves (8 with several blocks)."""
    n, k, m = 64, 512, 4
    c = Int4Case((_rng(900).standard_normal((n, k)) * 0.02).astype(np.float32), 128)
    tp = G.pack_tiled(G.W_INT4_ZP, c.d_packed, k, G.W_INT4_TILED_PAIRED, sc0=c.d_sz)
    t = G.pack_tiled(G.W_INT4_ZP, c.d_packed, k, G.W_INT4_TILED, sc0=c.d_sz)
    x = bf16_tensor(_x(m, k, 901))
    gamma = bf16_tensor(O.f32_to_bf16_bits(np.ones(k, np.float32)))
    cases = [
        (dict(w=tp, wfmt=G.W_INT4_TILED_PAIRED, epilogue=G.EPI_SILU_GATE), "status 4"),
        (dict(w=t, wfmt=G.W_INT4_TILED, gamma=gamma), "status 4"),
        (dict(w=t, wfmt=G.W_INT4_TILED, out2=torch.zeros(m, 16, device="cuda", dtype=torch.bfloat16)), "status 4"),
        (dict(w=t, wfmt=G.W_INT4_TILED, cfg=(0, 0, 6, PANEL)), "status 1"),
        (dict(w=t, wfmt=G.W_INT4_TILED, cfg=(0, 17, 1, PANEL)), "status 1"),
        (dict(w=t, wfmt=G.W_INT4_TILED, cfg=(0, 9, 2, PANEL)), "status 1"),
    ]
    for kw, code in cases:
        kw = dict(kw)
        w, wf = kw.pop("w"), kw.pop("wfmt")
        kw["cfg"] = kw.get("cfg", (0, 0, 0, PANEL))
        with pytest.raises(RuntimeError, match=code):
            G.gemv(x, w, wf, n, **kw)
    # row-major weights have no panel path
    with pytest.raises(RuntimeError, match="status 4"):
        G.gemv(x, c.d_packed, G.W_INT4_ZP, n, sc0=c.d_sz, cfg=(0, 0, 0, PANEL))


def test_panel_taken_without_a_workspace():
    """Through the C ABI with no workspace, several rows that the rule gives
    the tile kernel (K10240 at M = 32, which needs split-K partials) run on
    the panel kernel over the whole K instead: bit-identical to forcing path
    6 with one slice."""
    import ctypes

    from breeze_amd import _lib

    n, k, m = 2560, 10240, 32
    buf, wf, w_eff = _weight("int4", n, k, 1000)
    x = bf16_tensor(_x(m, k, 1001))
    out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    d = _lib.GemvDesc()
    d.abi_version = _lib.ABI_VERSION
    d.M, d.N, d.K, d.group, d.wfmt = m, n, k, 128, wf
    d.epilogue, d.out_dtype, d.residual_dtype = G.EPI_NONE, _lib.DT_BF16, _lib.DT_BF16
    d.eps = 1e-6
    d.x, d.ldx, d.w = x.data_ptr(), x.stride(0), buf.data_ptr()
    d.out, d.ldo = out.data_ptr(), out.stride(0)
    assert _lib.lib().bz_gemv_workspace(ctypes.byref(d)) > 0  # the rule's tile kernel would need one
    _lib.check(_lib.lib().bz_gemv(ctypes.byref(d), _lib.stream_of(x)), "bz_gemv")
    want = G.gemv(x, buf, wf, n, cfg=(0, 0, 0, PANEL, 1))
    assert torch.equal(out, want)
    assert O.rel_err(f32(out), _ref(_x(m, k, 1001), w_eff)) <= TIGHT


# ---------------------------------------------------------------------------
# K slices: fp32 sums per slice in the workspace, the last arrival of each
# row-block group adds them in slice order and applies the epilogue
# ---------------------------------------------------------------------------

SLICED = [
    # (fmt, n, k, m, blocks, slices)
    ("int4", 112, 1280, 9, 2, 3),      # 10 units / 3 slices: 4, 4, 2; a partial last group
    ("int4", 1024, 4096, 32, 3, 5),    # 32 units / 5: 7 x 4 + 4
    ("int4", 2560, 10240, 17, 1, 2),   # 16 waves x 3 units per slice
    ("fp8", 112, 1280, 9, 2, 3),       # 20 units / 3
    ("fp8", 1024, 4096, 32, 3, 4),
    ("fp8", 2560, 10240, 16, 5, 8),
]


@pytest.mark.parametrize("fmt,n,k,m,blocks,slices", SLICED, ids=[f"{c[0]}-N{c[1]}-K{c[2]}-M{c[3]}-T{c[4]}-S{c[5]}"
                                                                  for c in SLICED])
def test_panel_slices_match_oracle_and_whole_k(fmt, n, k, m, blocks, slices):
    buf, wf, w_eff = _weight(fmt, n, k, 1100 + slices, symmetric=(m % 2 == 1))
    x = _x(m, k, 1101 + m)
    res = _x(m, n, 1102) if slices % 2 else None
    out_dtype = torch.float32 if m == 17 else torch.bfloat16
    got = _run(buf, wf, n, x, cfg=(0, 0, blocks, PANEL, slices), res_bits=res, out_dtype=out_dtype)
    assert O.rel_err(f32(got), _ref(x, w_eff, res)) <= TIGHT
    # the same sums in another order (slice by slice): within one bf16 step
    # of the whole-K launch (one block per workgroup: up to 16 waves, enough
    # for every K here)
    whole = _run(buf, wf, n, x, cfg=(0, 0, 1, PANEL, 1), res_bits=res, out_dtype=out_dtype)
    assert O.rel_err(f32(got), f32(whole)) <= 2 ** -7
    # every call leaves the arrival counters zero: a second and third call are
    # bit-identical (a counter left non-zero would pick the wrong last arrival)
    for _ in range(2):
        assert torch.equal(_run(buf, wf, n, x, cfg=(0, 0, blocks, PANEL, slices), res_bits=res,
                                out_dtype=out_dtype), got)


@pytest.mark.parametrize(
    "fmt,n,k,m,blocks,slices",
    [
        ("int4", 2560, 10240, 32, 2, 3),   # the C4 down shape
        ("fp8", 2560, 10240, 32, 3, 4),
        ("fp8", 2560, 10240, 8, 3, 4),     # 160 KB of x
        ("int4", 2560, 10240, 12, 2, 3),
        ("fp8", 1024, 8192, 16, 1, 4),     # 64 blocks: one per workgroup
        ("int4", 1024, 8192, 32, 1, 4),
        ("fp8", 1024, 10240, 5, 1, 4),     # 100 KB of x, but only 64 blocks
        ("int4", 2560, 10240, 6, 5, 1),    # 120 KB of x: the whole K
        ("fp8", 2560, 4096, 32, 5, 1),     # K below 8192: the whole K
        ("int4", 20480, 2560, 32, 5, 1),   # K2560 N20480: the whole K, 5 blocks
    ],
)
def test_panel_rule_slices_at_full_size(fmt, n, k, m, blocks, slices):
    """The rule's K slices and blocks per workgroup are what the automatic
    call runs, bit for bit (with `blocks` = 5 and one slice standing for the
    whole-K plan, whose blocks per workgroup follow from N)."""
    buf, wf, w_eff = _weight(fmt, n, k, 1200)
    x = _x(m, k, 1201)
    auto = _run(buf, wf, n, x, cfg=(0, 0, 0, 0))
    if slices == 1:
        forced = _run(buf, wf, n, x, cfg=(0, 0, 0, PANEL, 1))
    else:
        forced = _run(buf, wf, n, x, cfg=(0, 0, blocks, PANEL, slices))
    assert torch.equal(auto, forced), (fmt, n, k, m)
    assert O.rel_err(f32(auto), _ref(x, w_eff)) <= TIGHT


def test_panel_slices_graph_replays_match_eager():
    n, k, m = 2560, 10240, 32
    buf, wf, _ = _weight("fp8", n, k, 1300)
    x = bf16_tensor(_x(m, k, 1301))
    out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
    call = lambda: G.gemv(x, buf, wf, n, out=out, cfg=(0, 0, 3, PANEL, 4))  # noqa: E731
    call()
    torch.cuda.synchronize()
    want = out.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side), torch.cuda.graph(g, stream=side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    for i in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), i
        _ = (x.float() * 2).sum().item()


def test_panel_forced_slices_need_the_workspace():
    """Through the C ABI: forced slices without a workspace are refused
    (status 1) and nothing runs; the workspace the library asks for makes the
    same call run."""
    import ctypes

    from breeze_amd import _lib

    n, k, m = 256, 2048, 8
    buf, wf, w_eff = _weight("int4", n, k, 1400)
    xb = _x(m, k, 1401)
    x = bf16_tensor(xb)
    out = torch.zeros(m, n, device="cuda", dtype=torch.bfloat16)
    d = _lib.GemvDesc()
    d.abi_version = _lib.ABI_VERSION
    d.M, d.N, d.K, d.group, d.wfmt = m, n, k, 128, wf
    d.epilogue, d.out_dtype, d.residual_dtype = G.EPI_NONE, _lib.DT_BF16, _lib.DT_BF16
    d.eps = 1e-6
    d.x, d.ldx, d.w = x.data_ptr(), x.stride(0), buf.data_ptr()
    d.out, d.ldo = out.data_ptr(), out.stride(0)
    d.cfg_path, d.cfg_tiles, d.cfg_slices = PANEL, 2, 4
    need = _lib.lib().bz_gemv_workspace(ctypes.byref(d))
    assert need == 16384 + 4 * m * n * 4
    assert _lib.lib().bz_gemv(ctypes.byref(d), _lib.stream_of(x)) == _lib.ERR_INVALID_ARG
    torch.cuda.synchronize()
    assert not out.any()
    ws = torch.zeros(need // 4, device="cuda", dtype=torch.int32)
    d.workspace, d.workspace_bytes = ws.data_ptr(), need
    _lib.check(_lib.lib().bz_gemv(ctypes.byref(d), _lib.stream_of(x)), "bz_gemv")
    assert O.rel_err(f32(out), _ref(xb, w_eff)) <= TIGHT
    assert not ws[:4096].any()  # the counters are left zero
