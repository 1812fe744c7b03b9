"""GPU parity of the several-row tile kernel (GEMV path 4: up to 32 rows of x
per launch, K sliced across workgroups, split-K partials summed in slice
order by the last workgroup of each column block) against the CPU oracle.

Bars as for the other GEMV paths: max|out-ref|/max|ref| <= 1e-2 against the
float64 dequantize-then-matmul of the same packed weights (bench_gemv.py:53)
and <= 4e-3 against the same-rounding oracle; one-hot x with dyadic scales
is bit-exact (pins the nibble order, the group index and the row/column
mapping of both operands and of the partials).
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

from breeze_amd import gemv as G  # noqa: E402

PATH = 4


def _res(M, n, seed):
    return O.f32_to_bf16_bits(np.random.default_rng(seed).standard_normal((M, n)).astype(np.float32))


def _case(fmt, N, K, seed, layout="zp"):
    """(call(x_bits, epi, res_bits, cfg, out_dtype) -> tensor, w_eff, row_scale)."""
    w, _, _ = O.synth(N, K, 1, seed=seed)
    if fmt == "int4":
        c = Int4Case(w, 128)
        if layout == "zp":
            kw = dict(sc0=c.d_sz, group=128)
            fmt_id, w_eff = G.W_INT4_ZP, c.w_zp
        else:
            kw = dict(sc0=c.d_s, sc1=c.d_m, group=128)
            fmt_id, w_eff = G.W_INT4_MIN, c.w_min
        wt, rs = c.d_packed, None
    elif fmt == "fp8":
        c = Fp8Case(w)
        kw = dict(sc0=c.d_scale)
        fmt_id, w_eff, wt, rs = G.W_FP8, O.e4m3fn_decode(c.codes), c.d_codes, c.scale
    else:
        wb = O.f32_to_bf16_bits(w)
        kw = {}
        fmt_id, w_eff, wt, rs = G.W_BF16, O.bf16_bits_to_f32(wb), bf16_tensor(wb), None

    def call(x_bits, epi=G.EPI_NONE, res_bits=None, cfg=(0, 0, 0, PATH), out_dtype=torch.bfloat16):
        return G.gemv(bf16_tensor(x_bits), wt, fmt_id, N, epilogue=epi,
                      residual=bf16_tensor(res_bits) if res_bits is not None else None, cfg=cfg,
                      out_dtype=out_dtype, **kw)

    return call, w_eff, rs


def _check(got, x_bits, w_eff, epi=O.EPI_NONE, res_bits=None, rs=None):
    x = O.bf16_bits_to_f32(x_bits)
    res = O.bf16_bits_to_f32(res_bits) if res_bits is not None else None
    ref = O.gemv_ref(x, w_eff, epi, res, rs)
    e = O.rel_err(f32(got), ref)
    assert e <= TIGHT, e
    return e


# Small shapes: ragged N (a partial column block and a partial 16-column tile),
# K = whole units of each format (int4 128 k, fp8 64 k, bf16 32 k).
SMALL = {"int4": (200, 1280), "fp8": (200, 1088), "bf16": (136, 544)}


@pytest.mark.parametrize("fmt,layout", [("int4", "zp"), ("int4", "min"), ("fp8", "zp"), ("bf16", "zp")])
@pytest.mark.parametrize("M", [1, 5, 8, 16, 17, 32])
@pytest.mark.parametrize("nsl", [0, 1, 3])
def test_tile_small(fmt, layout, M, nsl):
    N, K = SMALL[fmt]
    call, w_eff, rs = _case(fmt, N, K, seed=M + 3 * nsl, layout=layout)
    x = O.synth(8, K, M, seed=40 + M)[2]
    _check(call(x, cfg=(0, 0, 0, PATH, nsl)), x, w_eff, rs=rs)


@pytest.mark.parametrize("fmt", ["int4", "fp8", "bf16"])
@pytest.mark.parametrize("depth,waves,tiles,nsl", [(2, 4, 1, 2), (8, 8, 1, 5), (4, 4, 2, 0), (8, 8, 2, 7), (2, 8, 2, 1),
                                                   (4, 4, 1, 64), (4, 8, 1, 0)])
def test_tile_launch_shapes_residual(fmt, depth, waves, tiles, nsl):
    """Every (depth, waves, tiles, slices) shape, residual epilogue, fp32 and bf16 out."""
    N, K = SMALL[fmt]
    M = 20
    call, w_eff, rs = _case(fmt, N, K, seed=7)
    x = O.synth(8, K, M, seed=8)[2]
    res = _res(M, N, 9)
    for od in (torch.bfloat16, torch.float32):
        got = call(x, G.EPI_RESIDUAL, res, cfg=(depth, waves, tiles, PATH, nsl), out_dtype=od)
        _check(got, x, w_eff, O.EPI_RES, res, rs)


@pytest.mark.parametrize("fmt", ["int4", "fp8"])
@pytest.mark.parametrize("M", [33, 70])
def test_tile_more_than_32_rows(fmt, M):
    """M > 32: one launch per 32 rows (the last one shorter)."""
    N, K = SMALL[fmt]
    call, w_eff, rs = _case(fmt, N, K, seed=11)
    x = O.synth(8, K, M, seed=12)[2]
    res = _res(M, N, 13)
    _check(call(x, G.EPI_RESIDUAL, res, cfg=(0, 0, 0, PATH, 3)), x, w_eff, O.EPI_RES, res, rs)
    _check(call(x, G.EPI_NONE, cfg=(0, 0, 0, 0)), x, w_eff, rs=rs)  # automatic rule


def test_tile_counters_reset_and_deterministic():
    """Split-K calls in a row (counters left at zero by each call) give
    bit-identical outputs; a different shape in between does not disturb
    the next call."""
    call, w_eff, _ = _case("int4", 200, 1280, seed=14)
    x = O.synth(8, 1280, 24, seed=15)[2]
    first = call(x, cfg=(0, 0, 0, PATH, 5)).clone()
    _check(first, x, w_eff)
    call2, w2, rs2 = _case("fp8", 136, 1088, seed=16)
    x2 = O.synth(8, 1088, 9, seed=17)[2]
    _check(call2(x2, cfg=(0, 0, 0, PATH, 17)), x2, w2, rs=rs2)
    for _ in range(3):
        again = call(x, cfg=(0, 0, 0, PATH, 5))
        assert torch.equal(again, first)


def test_tile_one_hot_int4_bit_exact():
    """x = e_k with dyadic scales: every output is exactly w_eff[:, k], also
    through the split-K partials."""
    N, K, group = 80, 1024, 128
    rng = np.random.default_rng(18)
    q = rng.integers(0, 16, (N, K), dtype=np.uint8)
    s = (2.0 ** rng.integers(-8, -4, (N, K // group))).astype(np.float32)
    z = (rng.integers(-64, 64, (N, K // group)) * 2.0 ** -9).astype(np.float32)
    sz = O.scales_zeros(s, z)
    w_eff = O.dequant_int4_zp(q, sz, group)
    d_w, d_sz = u8_tensor(O.pack_nibbles_even_low(q)), bf16_tensor(sz)
    ks = list(range(0, K, 33))[:32]
    x = np.zeros((len(ks), K), np.float32)
    x[np.arange(len(ks)), ks] = 1.0
    for nsl in (1, 3, 8):
        got = f32(G.gemv(bf16_tensor(O.f32_to_bf16_bits(x)), d_w, G.W_INT4_ZP, N, sc0=d_sz, group=group,
                         out_dtype=torch.float32, cfg=(0, 0, 0, PATH, nsl)))
        for i, k in enumerate(ks):
            assert np.array_equal(got[i], w_eff[:, k]), (nsl, k)


def test_tile_one_hot_fp8_bit_exact():
    N, K = 80, 512
    rng = np.random.default_rng(19)
    codes = rng.integers(0, 256, (N, K), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x10          # no NaN codes
    want = O.e4m3fn_decode(codes)
    ks = [0, 1, 2, 7, 8, 15, 16, 31, 32, 63, 64, 65, 100, 255, 256, 300, 447, 448, 500, 511]
    x = np.zeros((len(ks), K), np.float32)
    x[np.arange(len(ks)), ks] = 1.0
    for nsl in (1, 4):
        got = f32(G.gemv(bf16_tensor(O.f32_to_bf16_bits(x)), u8_tensor(codes), G.W_FP8, N,
                         sc0=torch.ones(N, device="cuda"), out_dtype=torch.float32, cfg=(0, 0, 0, PATH, nsl)))
        for i, k in enumerate(ks):
            assert np.array_equal(got[i], want[:, k]), (nsl, k)


@pytest.mark.parametrize("fmt", ["int4", "fp8"])
@pytest.mark.parametrize("N,K", [(20480, 2560), (2560, 10240)])
def test_tile_full_size(fmt, N, K):
    """The several-row shapes of the benchmark (M = 32, automatic rule)
    against the float64 reference (bar 1e-2) and the same-rounding oracle."""
    M = 32
    call, w_eff, rs = _case(fmt, N, K, seed=20)
    x = O.synth(8, K, M, seed=21)[2]
    got = call(x, cfg=(0, 0, 0, 0))
    e = _check(got, x, w_eff, rs=rs)
    assert e <= TOL


def test_tile_path_rejects_what_it_cannot_run():
    call, _, _ = _case("int4", 200, 1280, seed=22)
    x = O.synth(8, 1280, 8, seed=23)[2]
    with pytest.raises(RuntimeError, match="exceeds what this build supports"):
        call(x, G.EPI_SILU_GATE, cfg=(0, 0, 0, PATH))
    with pytest.raises(RuntimeError, match="invalid argument"):
        call(x, cfg=(3, 0, 0, PATH))    # depth 3
    with pytest.raises(RuntimeError, match="invalid argument"):
        call(x, cfg=(0, 0, 3, PATH))    # 3 tiles per wave
    with pytest.raises(RuntimeError, match="invalid argument"):
        call(x, cfg=(0, 5, 0, PATH))    # 5 waves per workgroup


def test_tile_graph_replays_match_eager():
    """A captured split-K tile GEMV replayed several times, with eager work
    and synchronizations in between, equals the eager result every time."""
    x_bits = O.synth(8, 1280, 16, seed=25)[2]
    x = bf16_tensor(x_bits)
    c = Int4Case(O.synth(200, 1280, 1, seed=24)[0], 128)
    out = torch.empty(16, 200, device="cuda", dtype=torch.bfloat16)

    def run():
        G.gemv(x, c.d_packed, G.W_INT4_ZP, 200, sc0=c.d_sz, group=128, out=out, cfg=(0, 0, 0, PATH, 5))

    run()
    torch.cuda.synchronize()
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s), torch.cuda.graph(g, stream=s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    for i in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        _ = (x.float() * 2).sum()     # unrelated eager work between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("fmt", ["int4", "fp8", "bf16"])
@pytest.mark.parametrize("depth", [2, 4, 8])
@pytest.mark.parametrize("tiles", [1, 2])
@pytest.mark.parametrize("M", [8, 24])
@pytest.mark.parametrize("waves", [4, 8])
def test_tile_every_instance_steady_loop(fmt, depth, tiles, M, waves):
    """Every (depth, tiles, row blocks) instance with one slice of >= 16
    units, so the unrolled steady loop of the weight pipeline runs (the
    first unit comes from the prologue's loads).  Regression: the nibble
    unpack that feeds the MFMA B operand once came from inline assembly,
    which the compiler's hazard pass does not see, and the int4 instance with
    depth 4, 2 tiles and one row block read a B register one instruction
    after it was written (wrong second tile of every wave in the first unit)."""
    N, K = {"int4": (160, 2560), "fp8": (160, 1024), "bf16": (160, 512)}[fmt]
    call, w_eff, rs = _case(fmt, N, K, seed=30 + depth + tiles + M)
    x = O.synth(8, K, M, seed=31)[2]
    _check(call(x, cfg=(depth, waves, tiles, PATH, 1), out_dtype=torch.float32), x, w_eff, rs=rs)


def _ws_key(stream: torch.cuda.Stream, capture=None):
    return (torch.cuda.current_device(), stream.cuda_stream, capture)


def test_tile_graph_survives_workspace_growth():
    """A graph captured over a tile-path GEMV gets a workspace of its own
    (allocated from the graph's pool, its zero fill recorded in the graph),
    and keeps working after an eager call on the capture stream has grown
    (replaced) that stream's workspace: the outgrown buffer stays alive."""
    from breeze_amd import gemv as gemv_mod

    c = Int4Case(O.synth(200, 1280, 1, seed=26)[0], 128)
    x = bf16_tensor(O.synth(8, 1280, 16, seed=27)[2])
    out = torch.empty(16, 200, device="cuda", dtype=torch.bfloat16)

    def run():
        G.gemv(x, c.d_packed, G.W_INT4_ZP, 200, sc0=c.d_sz, group=128, out=out, cfg=(0, 0, 0, PATH, 5))

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        gemv_mod._GEMV_WS.pop(_ws_key(s), None)  # start from a fresh (small) workspace on s
        run()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    eager = out.clone()
    before = gemv_mod._GEMV_WS[_ws_key(s)]
    n_graph = sum(1 for k in gemv_mod._GEMV_WS if k[2] is not None)
    g = torch.cuda.CUDAGraph()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s), torch.cuda.graph(g, stream=s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    graph_bufs = [v for k, v in gemv_mod._GEMV_WS.items() if k[2] is not None]
    assert len(graph_bufs) == n_graph + 1  # the capture's own workspace
    assert all(b.data_ptr() != before.data_ptr() for b in graph_bufs)
    # a split-K call on s needing more than the fresh 1 MiB workspace grows s's
    big = Int4Case(O.synth(2048, 2560, 1, seed=28)[0], 128)
    xb_bits = O.synth(8, 2560, 32, seed=29)[2]
    assert 20 * 32 * 2048 * 4 > before.numel() * 4
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        got = G.gemv(bf16_tensor(xb_bits), big.d_packed, G.W_INT4_ZP, 2048, sc0=big.d_sz, group=128,
                     cfg=(0, 0, 0, PATH, 20))
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert gemv_mod._GEMV_WS[_ws_key(s)].data_ptr() != before.data_ptr()
    _check(got, xb_bits, big.w_zp)
    for i in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        run()  # eager work on the current stream between the replays
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i


def test_tile_two_streams_own_workspaces():
    """Split-K tile GEMVs issued on two streams at once: each stream uses a
    workspace of its own (different buffers), and both results equal the
    ones the same calls give one after the other on one stream."""
    from breeze_amd import gemv as gemv_mod

    N, K, M = 2560, 10240, 32
    cases = [Int4Case(O.synth(N, K, 1, seed=40 + i)[0], 128) for i in range(2)]
    xs = [bf16_tensor(O.synth(8, K, M, seed=42 + i)[2]) for i in range(2)]

    def call(i):
        return G.gemv(xs[i], cases[i].d_packed, G.W_INT4_ZP, N, sc0=cases[i].d_sz, group=128,
                      cfg=(0, 0, 0, PATH, 10))

    serial = [call(0), call(1)]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in range(2)]
    outs = [None, None]
    for rep in range(4):
        for i, st in enumerate(streams):
            st.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(st):
                outs[i] = call(i)
        for st in streams:
            torch.cuda.current_stream().wait_stream(st)
        torch.cuda.synchronize()
        assert torch.equal(outs[0], serial[0]) and torch.equal(outs[1], serial[1]), rep
    bufs = [gemv_mod._GEMV_WS[_ws_key(st)] for st in streams]
    assert bufs[0].data_ptr() != bufs[1].data_ptr()
    _check(outs[0], O.f32_to_bf16_bits(xs[0].float().cpu().numpy()), cases[0].w_zp)


@pytest.mark.parametrize("fmt", ["int4", "fp8"])
def test_tile_fp32_residual_aliasing_out(fmt):
    """Residual epilogue with an fp32 residual that is also the output
    (in-place residual add, which the C ABI allows), several slices."""
    N, K = SMALL[fmt]
    M = 10
    _, w_eff, rs = _case(fmt, N, K, seed=32)
    x = O.synth(8, K, M, seed=33)[2]
    res = np.random.default_rng(34).standard_normal((M, N)).astype(np.float32)
    buf = torch.from_numpy(res.copy()).cuda()
    w, _, _ = O.synth(N, K, 1, seed=32)
    if fmt == "int4":
        c = Int4Case(w, 128)
        G.gemv(bf16_tensor(x), c.d_packed, G.W_INT4_ZP, N, sc0=c.d_sz, group=128, epilogue=G.EPI_RESIDUAL,
               residual=buf, out=buf, cfg=(0, 0, 0, PATH, 4))
    else:
        c = Fp8Case(w)
        G.gemv(bf16_tensor(x), c.d_codes, G.W_FP8, N, sc0=c.d_scale, epilogue=G.EPI_RESIDUAL, residual=buf,
               out=buf, cfg=(0, 0, 0, PATH, 4))
    ref = O.gemv_ref(O.bf16_bits_to_f32(x), w_eff, O.EPI_RES, res, rs)
    assert O.rel_err(f32(buf), ref) <= TIGHT
