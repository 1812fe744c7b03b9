"""GPU tests of the reference-shaped modules and of the committed golden
fixtures, all through the C ABI (libbzgemv.so).

Bars: bit-exact for quantizer outputs, packing and dequantized weights;
max|out-ref|/max|ref| <= 1e-2 for GEMV outputs against the CPU oracle's
float64 product on the fp32 RMSNorm (the reference's own definition,
bench_gemv.py:30-53)."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch
from torch import nn

from oracle import bz_oracle as O
from tests._util import bf16_bits, bf16_tensor, f32, u8_tensor

from breeze_amd import fp8_linear as F8
from breeze_amd import gemv as G
from breeze_amd import int4_linear as I4
from breeze_amd.fused import kernels as FK

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
TOL = 1e-2


def _dev():
    return torch.device("cuda", 0)


# ---------------------------------------------------------------------------
# golden fixtures
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("name", ["int4_asym_g128", "int4_sym_g128", "int4_asym_g32"])
def test_golden_int4(name):
    f = np.load(GOLDEN / f"{name}.npz")
    n, k, m, group, sym = (int(v) for v in f["meta"])
    # quantizer: bit-exact packed bytes and scales_zeros
    packed, sz, _ = G.quantize_int4_device(torch.from_numpy(f["w"]).to(_dev()), group, bool(sym), G.W_INT4_ZP)
    assert np.array_equal(packed.cpu().numpy(), f["packed_even_low"])
    assert np.array_equal(bf16_bits(sz), f["scales_zeros"])
    if not sym:
        p2, s2, m2 = G.quantize_int4_device(torch.from_numpy(f["w"]).to(_dev()), group, False, G.W_INT4_MIN)
        assert np.array_equal(p2.cpu().numpy(), f["packed_even_low"])
        assert np.array_equal(bf16_bits(s2), f["scale_bits"]) and np.array_equal(bf16_bits(m2), f["min_bits"])
    # dequant: bit-exact in both scale layouts
    d_p = u8_tensor(f["packed_even_low"])
    got = G.dequant(G.W_INT4_ZP, d_p, n, k, sc0=bf16_tensor(f["scales_zeros"]), group=group)
    assert np.array_equal(got.cpu().numpy(), f["w_eff_zp"])
    got = G.dequant(G.W_INT4_MIN, d_p, n, k, sc0=bf16_tensor(f["scale_bits"]), sc1=bf16_tensor(f["min_bits"]),
                    group=group)
    assert np.array_equal(got.cpu().numpy(), f["w_eff_min"])
    # GEMVs against the stored float64 references
    x, g = bf16_tensor(f["x"]), bf16_tensor(f["gamma"])
    sz_d = bf16_tensor(f["scales_zeros"])
    for path in (1, 2):
        if path == 2 and group < 128:
            continue
        cfg = (0, 0, 0, path)
        out = G.gemv(x, d_p, G.W_INT4_ZP, n, sc0=sz_d, group=group, gamma=g, out_dtype=torch.float32, cfg=cfg)
        assert O.rel_err(f32(out), f["out_norm_none"]) <= TOL
        out = G.gemv(x, d_p, G.W_INT4_ZP, n, sc0=sz_d, group=group, gamma=g, epilogue=G.EPI_SILU_GATE, cfg=cfg)
        assert O.rel_err(f32(out), f["out_norm_silu"]) <= TOL
        out = G.gemv(x, d_p, G.W_INT4_ZP, n, sc0=sz_d, group=group, epilogue=G.EPI_RESIDUAL,
                     residual=bf16_tensor(f["residual"]), cfg=cfg)
        assert O.rel_err(f32(out), f["out_plain_res"]) <= TOL
        out = G.gemv(x, d_p, G.W_INT4_MIN, n, sc0=bf16_tensor(f["scale_bits"]), sc1=bf16_tensor(f["min_bits"]),
                     group=group, cfg=cfg)
        assert O.rel_err(f32(out), f["out_min_none"]) <= TOL


def test_golden_fp8():
    f = np.load(GOLDEN / "fp8_row.npz")
    n, k, m = (int(v) for v in f["meta"])
    w = torch.from_numpy(f["w"]).to(_dev())
    codes, scale = G.quantize_fp8_device(w, 1e-12)
    assert np.array_equal(codes.view(torch.uint8).cpu().numpy(), f["codes"])
    assert np.array_equal(scale.cpu().numpy(), f["scale"])
    c8, s8 = G.quantize_fp8_device(w, 1e-8)
    assert np.array_equal(c8.view(torch.uint8).cpu().numpy(), f["codes_fused"])
    assert np.array_equal(s8.cpu().numpy(), f["scale_fused"])
    d_c = u8_tensor(f["codes"])
    d_s = torch.from_numpy(f["scale"]).to(_dev())
    # decoded codes times the row scale is bit-exact
    got = G.dequant(G.W_FP8, d_c, n, k, sc0=d_s)
    assert np.array_equal(got.cpu().numpy(), f["w_eff"])
    x, g = bf16_tensor(f["x"]), bf16_tensor(f["gamma"])
    for path in (1, 2):
        out = G.gemv(x, d_c, G.W_FP8, n, sc0=d_s, gamma=g, out_dtype=torch.float32, cfg=(0, 0, 0, path))
        assert O.rel_err(f32(out), f["out_norm_none"]) <= TOL
        out = G.gemv(x, d_c, G.W_FP8, n, sc0=d_s, epilogue=G.EPI_SILU_GATE, cfg=(0, 0, 0, path))
        assert O.rel_err(f32(out), f["out_plain_silu"]) <= TOL


# ---------------------------------------------------------------------------
# Int4Linear / Fp8Linear (models/int4_linear.py:67-115, models/fp8_linear.py:44-86)
# ---------------------------------------------------------------------------


def _linear(n, k, seed, device):
    w, _, _ = O.synth(n, k, 1, seed=seed)
    lin = nn.Linear(k, n, bias=False)
    with torch.no_grad():
        lin.weight.copy_(torch.from_numpy(w))
    return lin.to(device), w


@pytest.mark.parametrize("device", ["cuda", "cpu"])
def test_int4_linear_buffers_and_forward(device):
    N, K = 384, 1024
    lin, w = _linear(N, K, 20, device)
    mod = I4.Int4Linear(lin, device="cuda" if device == "cpu" else None)
    assert mod.in_features == K and mod.out_features == N and mod.group_size == 128
    assert mod.weight_int4.dtype == torch.int32 and tuple(mod.weight_int4.shape) == I4.tiled_shape(N, K)
    assert mod.scales_zeros.dtype == torch.bfloat16 and tuple(mod.scales_zeros.shape) == (K // 128, N, 2)
    q, s, lo, z = O.quantize_int4_asym(w, 128)
    sz = O.scales_zeros(s, z)
    assert np.array_equal(bf16_bits(mod.scales_zeros), sz)
    tiled = O.tile_int4(O.pack_nibbles_even_low(q), sz)
    assert np.array_equal(mod.weight_int4.cpu().view(torch.uint8).numpy().reshape(-1), tiled)
    w_eff = O.dequant_int4_zp(q, sz, 128)
    # M = 1..12 on the streaming kernel (slices of <= 8 rows); 40 and 100 on the prefill branch
    for shape, dtype in (((1, K), torch.bfloat16), ((2, 3, K), torch.bfloat16), ((5, K), torch.float32),
                         ((2, 6, K), torch.bfloat16), ((40, K), torch.bfloat16), ((100, K), torch.float32)):
        x = torch.randn(*shape, generator=torch.Generator().manual_seed(3)).to(dtype)
        y = mod(x.to(_dev()))
        assert y.dtype == dtype and tuple(y.shape) == shape[:-1] + (N,)
        xr = x.to(torch.bfloat16).float().reshape(-1, K).numpy()
        assert O.rel_err(f32(y).reshape(-1, N), O.gemv_ref(xr, w_eff)) <= TOL


@pytest.mark.parametrize("group", [32, 64])
def test_int4_linear_rowmajor_groups(group):
    """Groups other than 128 keep the row-major layout and its kernels, at
    decode and several-row M (an int4 table entry forcing a path that needs
    group 128 must give way to the built-in rule)."""
    N, K = 2560, 1024
    lin, w = _linear(N, K, 23 + group, "cuda")
    mod = I4.Int4Linear(lin, group_size=group)
    assert tuple(mod.weight_int4.shape) == (N, K // 8)
    assert I4.layout_of(mod.weight_int4, N, K) == I4.LAYOUT_ROWMAJOR
    q, s, lo, z = O.quantize_int4_asym(w, group)
    assert np.array_equal(mod.weight_int4.cpu().view(torch.uint8).numpy(), O.pack_nibbles_even_low(q))
    w_eff = O.dequant_int4_zp(q, O.scales_zeros(s, z), group)
    for M in (1, 2, 4, 16):
        x = torch.randn(M, K, generator=torch.Generator().manual_seed(M)).to(torch.bfloat16)
        y = mod(x.to(_dev()))
        assert O.rel_err(f32(y), O.gemv_ref(x.float().numpy(), w_eff)) <= TOL, M


def test_int4_linear_retile():
    """A row-major module of a tileable shape, re-tiled in place, computes
    the same product (the checkpoint loader's conversion of row-major files)."""
    N, K = 512, 1024
    lin, w = _linear(N, K, 24, "cuda")
    ref = I4.Int4Linear(lin)
    q, s, lo, z = O.quantize_int4_asym(w, 128)
    mod = I4.Int4Linear.__new__(I4.Int4Linear)
    nn.Module.__init__(mod)
    mod.in_features, mod.out_features, mod.group_size = K, N, 128
    mod.register_buffer("weight_int4", torch.from_numpy(O.pack_nibbles_even_low(q)).view(torch.int32).cuda())
    mod.register_buffer("scales_zeros", ref.scales_zeros.clone())
    x = torch.randn(2, K, device=_dev()).to(torch.bfloat16)
    before = mod(x)
    assert I4.retile(mod) and not I4.retile(mod)
    assert torch.equal(mod.weight_int4, ref.weight_int4)
    assert torch.equal(mod(x), ref(x))
    assert O.rel_err(f32(before), f32(ref(x))) <= 2.0 ** -7


def test_int4_linear_rebuilt_from_buffers():
    """The quantized-checkpoint loader builds modules with __new__ +
    nn.Module.__init__ + attributes + register_buffer
    (models/quantized_checkpoint.py:91-107); forward must need nothing else."""
    N, K = 256, 512
    lin, w = _linear(N, K, 21, "cuda")
    ref = I4.Int4Linear(lin)
    mod = I4.Int4Linear.__new__(I4.Int4Linear)
    nn.Module.__init__(mod)
    mod.in_features, mod.out_features, mod.group_size = K, N, 128
    mod.register_buffer("weight_int4", ref.weight_int4.clone())
    mod.register_buffer("scales_zeros", ref.scales_zeros.clone())
    x = torch.randn(2, K, device=_dev()).to(torch.bfloat16)
    assert torch.equal(mod(x), ref(x))


def _fp8_codes(mod):
    """(codes uint8 [N, K], scales [N]) of an Fp8Linear in either layout."""
    if F8.layout_of(mod.weight_fp8, mod.out_features, mod.in_features) == F8.LAYOUT_ROWMAJOR:
        return mod.weight_fp8.view(torch.uint8).cpu().numpy(), mod.weight_scale.cpu().numpy()[0]
    return O.untile_fp8(mod.weight_fp8.view(torch.uint8).cpu().numpy().reshape(-1), mod.out_features,
                        mod.in_features)


def test_fp8_linear_buffers_and_forward():
    """A tileable shape: weight_fp8 holds the tiled bytes (the oracle's tiling
    of the reference-formula codes and scales, byte for byte), weight_scale
    the reference's (1, N) scales; forward runs the tiled GEMV paths and, past
    32 rows, the chunked dequantize-then-GEMM."""
    N, K = 320, 768
    lin, w = _linear(N, K, 22, "cuda")
    mod = F8.Fp8Linear(lin)
    assert mod.weight_fp8.dtype == torch.float8_e4m3fn
    assert tuple(mod.weight_fp8.shape) == F8.tiled_shape(N, K) == (N // 16, 16 * K + 128)
    assert F8.layout_of(mod.weight_fp8, N, K) == F8.LAYOUT_TILED
    assert mod.weight_scale.dtype == torch.float32 and tuple(mod.weight_scale.shape) == (1, N)
    codes, scale = O.quantize_fp8_linear(w)
    assert np.array_equal(mod.weight_fp8.view(torch.uint8).cpu().numpy().reshape(-1), O.tile_fp8(codes, scale))
    assert np.array_equal(mod.weight_scale.cpu().numpy()[0], scale)
    for M in (1, 2, 3, 12, 40):  # streaming, panel, chunked dequantize-then-GEMM
        x = torch.randn(M, K, device=_dev()).to(torch.bfloat16)
        y = mod(x)
        assert y.dtype == torch.bfloat16 and tuple(y.shape) == (M, N)
        ref = O.gemv_ref(x.float().cpu().numpy(), O.dequant_fp8(codes, scale))
        assert O.rel_err(f32(y), ref) <= TOL, M


def test_fp8_linear_rowmajor_buffers_retile():
    """A module holding the reference's row-major buffers (as its checkpoints
    do) gives the same outputs before and after retile(), which turns it into
    the tiled module's bytes."""
    N, K = 256, 1024
    lin, w = _linear(N, K, 23, "cuda")
    tiled = F8.Fp8Linear(lin)
    codes, scale = O.quantize_fp8_linear(w)
    mod = F8.Fp8Linear.__new__(F8.Fp8Linear)
    nn.Module.__init__(mod)
    mod.in_features, mod.out_features = K, N
    mod.register_buffer("weight_fp8", u8_tensor(codes).view(torch.float8_e4m3fn))
    mod.register_buffer("weight_scale", torch.from_numpy(scale.reshape(1, N).copy()).to(_dev()))
    x = torch.randn(2, K, device=_dev()).to(torch.bfloat16)
    before = mod(x)
    assert O.rel_err(f32(before), O.gemv_ref(x.float().cpu().numpy(), O.dequant_fp8(codes, scale))) <= TOL
    assert F8.retile(mod) and not F8.retile(mod)
    assert torch.equal(mod.weight_fp8.view(torch.uint8), tiled.weight_fp8.view(torch.uint8))
    assert torch.equal(mod(x), tiled(x))


@pytest.mark.parametrize("mod_kind", ["int4", "fp8"])
def test_prefill_rows_chunked(mod_kind):
    """More than 32 rows: the weight is decoded in runs of whole 16-row blocks
    (a 1 MiB fp32 budget here forces several runs, one of them short) and
    multiplied by the library GEMM; the result equals the one-run product."""
    N, K, M = 400, 1280, 48
    lin, w = _linear(N, K, 24, "cuda")
    mod = I4.Int4Linear(lin) if mod_kind == "int4" else F8.Fp8Linear(lin)
    buf = mod.weight_int4 if mod_kind == "int4" else mod.weight_fp8.view(torch.uint8)
    wfmt = G.W_INT4_TILED if mod_kind == "int4" else G.W_FP8_TILED
    x = torch.randn(M, K, device=_dev()).to(torch.bfloat16)
    small = G.dequant_matmul(x, buf, wfmt, N, K, chunk_bytes=1 << 20)   # 192-row runs: 192 + 192 + 16
    whole = G.dequant_matmul(x, buf, wfmt, N, K, chunk_bytes=1 << 30)
    assert torch.equal(small, whole)
    assert torch.equal(mod(x), whole)
    w_eff = f32(G.dequant(wfmt, buf, N, K))
    assert O.rel_err(f32(whole), O.gemv_ref(x.float().cpu().numpy(), w_eff)) <= TOL


class _Mlp(nn.Module):
    def __init__(self, k, n):
        super().__init__()
        self.gate_proj = nn.Linear(k, n, bias=False)
        self.up_proj = nn.Linear(k, n, bias=False)
        self.down_proj = nn.Linear(n, k, bias=False)

    def forward(self, x):
        return self.down_proj(torch.nn.functional.silu(self.gate_proj(x)) * self.up_proj(x))


def test_quantize_module_int4_converts_large_layers():
    torch.manual_seed(0)
    m = _Mlp(2048, 1536).to(_dev())          # 12 MB fp32 each: above the 8 MB threshold
    for p in m.parameters():
        nn.init.normal_(p, std=0.02)
    x = torch.randn(2, 2048, device=_dev())
    want = m(x)
    nbytes = 2048 * 1536 * 4
    stats = I4.quantize_module_int4(m)
    assert stats == {"converted": 3, "skipped_below_threshold": 0, "skipped_unsupported": 0,
                     "weight_bytes_saved": 3 * (nbytes - nbytes // 4)}
    assert all(type(getattr(m, n)) is I4.Int4Linear for n in ("gate_proj", "up_proj", "down_proj"))
    got = m(x)
    assert got.dtype == torch.float32
    # against the same MLP on the dequantized weights (decode pinned bit-exact
    # by the golden tests), fp32: only the kernel's bf16 activations differ
    wd = {n: G.dequant(G.W_INT4_TILED, getattr(m, n).weight_int4, getattr(m, n).out_features,
                       getattr(m, n).in_features)
          for n in ("gate_proj", "up_proj", "down_proj")}
    h = torch.nn.functional.silu(x @ wd["gate_proj"].t()) * (x @ wd["up_proj"].t())
    assert O.rel_err(f32(got), f32(h @ wd["down_proj"].t())) <= TOL
    # and the quantization error itself stays at int4 group-128 level
    assert O.rel_err(f32(got), f32(want)) <= 0.35


def test_quantize_module_fp8_converts_large_layers():
    torch.manual_seed(1)
    m = _Mlp(2048, 1536).to(_dev())
    for p in m.parameters():
        nn.init.normal_(p, std=0.02)
    x = torch.randn(2, 2048, device=_dev())
    want = m(x)
    stats = F8.quantize_module_fp8(m)
    nbytes = 2048 * 1536 * 4
    assert stats == {"converted": 3, "skipped_below_threshold": 0, "weight_bytes_saved": 3 * (nbytes // 2)}
    got = m(x)
    wd = {n: G.dequant(G.W_FP8_TILED, getattr(m, n).weight_fp8.view(torch.uint8), getattr(m, n).out_features,
                       getattr(m, n).in_features)
          for n in ("gate_proj", "up_proj", "down_proj")}
    h = torch.nn.functional.silu(x @ wd["gate_proj"].t()) * (x @ wd["up_proj"].t())
    assert O.rel_err(f32(got), f32(h @ wd["down_proj"].t())) <= TOL
    assert O.rel_err(f32(got), f32(want)) <= 0.1


# ---------------------------------------------------------------------------
# fused/ host API (models/fused/kernels.py, models/fused/layer.py)
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("bits", [4, 8, 16])
@pytest.mark.parametrize("epi", [0, 1, 2])
def test_rms_gemv(bits, epi):
    N, K, M = 512, 1024, 2
    w, gamma, x = O.synth(N, K, M, seed=30 + bits + epi)
    fw = FK.FusedWeight(torch.from_numpy(w).to(_dev()), bits=bits, paired=epi == 1)
    xd, gd = bf16_tensor(x), bf16_tensor(gamma)
    n_out = N // 2 if epi == 1 else N
    res = torch.randn(M, n_out, device=_dev()).to(torch.bfloat16) if epi == 2 else None
    out = FK.rms_gemv(xd, fw, gd, 1e-6, epilogue=epi, residual=res)
    if bits == 4:
        q = O.unpack_nibbles_even_low(fw.w.cpu().numpy())
        w_eff = O.dequant_int4_min(q, bf16_bits(fw.s), bf16_bits(fw.z), 128)
        packed, s_bits, m_bits = O.pack_int4_fused(w)
        assert np.array_equal(fw.w.cpu().numpy(), packed)           # pack_int4 bit-exact
        assert np.array_equal(bf16_bits(fw.s), s_bits) and np.array_equal(bf16_bits(fw.z), m_bits)
    elif bits == 8:
        codes, scale = O.pack_fp8(w)
        assert fw.layout == ("tiled-paired" if epi == 1 else "tiled") and fw.s is None
        assert np.array_equal(fw.w.cpu().numpy(), O.tile_fp8(codes, scale, paired=epi == 1))
        w_eff = O.dequant_fp8(codes, scale)
    else:
        w_eff = O.round_bf16(w)
    xn = O.rmsnorm_f32(O.bf16_bits_to_f32(x), O.bf16_bits_to_f32(gamma))
    ref = O.gemv_ref(xn, w_eff, epi, res.float().cpu().numpy() if res is not None else None)
    assert tuple(out.shape) == (M, n_out)
    assert O.rel_err(f32(out), ref) <= TOL


@pytest.mark.parametrize("paired", [True, False])
def test_from_int4_gate_up_silu(paired):
    """Two Int4Linear modules fused as [gate; up] with the SiLU-gate epilogue
    (models/fused/layer.py:56-60, kernels.py:116-127): one launch over the
    paired tiling, or GEMV + silu_mul over the unpaired one."""
    K, H = 1024, 384
    g_lin, wg = _linear(H, K, 40, "cuda")
    u_lin, wu = _linear(H, K, 41, "cuda")
    gm, um = I4.Int4Linear(g_lin), I4.Int4Linear(u_lin)
    fw = FK.FusedWeight.from_int4(gm, um, paired=paired)
    assert fw.N == 2 * H and fw.K == K and fw.layout == ("tiled-paired" if paired else "tiled")
    qg, sg, _, zg = O.quantize_int4_asym(wg, 128)
    qu, su, _, zu = O.quantize_int4_asym(wu, 128)
    sz = np.concatenate([O.scales_zeros(sg, zg), O.scales_zeros(su, zu)], axis=1)
    packed = O.pack_nibbles_even_low(np.concatenate([qg, qu]))
    assert np.array_equal(fw.w.cpu().numpy(), O.tile_int4(packed, sz, paired=paired))
    _, gamma, x = O.synth(1, K, 2, seed=42)
    out = FK.rms_gemv(bf16_tensor(x), fw, bf16_tensor(gamma), 1e-6, epilogue=FK.EPI_SILU_GATE)
    xn = O.rmsnorm_f32(O.bf16_bits_to_f32(x), O.bf16_bits_to_f32(gamma))
    w_eff = np.concatenate([O.dequant_int4_zp(qg, O.scales_zeros(sg, zg)), O.dequant_int4_zp(qu, O.scales_zeros(su, zu))])
    assert O.rel_err(f32(out), O.gemv_ref(xn, w_eff, O.EPI_SILU)) <= TOL
    if paired:
        with pytest.raises(ValueError, match="paired"):
            FK.rms_gemv(bf16_tensor(x), fw, bf16_tensor(gamma), 1e-6)


def test_from_int4_rowmajor_groups_concat():
    """Int4Linear modules of group 64 (row-major) are concatenated as they are."""
    K, H = 1024, 256
    mods = [I4.Int4Linear(_linear(H, K, 43 + i, "cuda")[0], group_size=64) for i in range(2)]
    fw = FK.FusedWeight.from_int4(*mods)
    assert fw.layout == "zp" and fw.group == 64
    x = torch.randn(2, K, device=_dev()).to(torch.bfloat16)
    out = FK.rms_gemv(x, fw)
    want = torch.cat([m(x) for m in mods], dim=1)
    assert O.rel_err(f32(out), f32(want)) <= 1e-2


@pytest.mark.parametrize("paired", [False, True])
def test_from_fp8_concat(paired):
    K = 768
    sizes = (256, 256) if paired else (256, 64, 64)
    mods = [F8.Fp8Linear(_linear(n, K, 50 + i, "cuda")[0]) for i, n in enumerate(sizes)]
    fw = FK.FusedWeight.from_fp8(*mods, paired=paired)
    assert fw.N == sum(sizes) and fw.layout == ("tiled-paired" if paired else "tiled")
    codes = np.concatenate([_fp8_codes(m)[0] for m in mods])
    scale = np.concatenate([_fp8_codes(m)[1] for m in mods])
    assert np.array_equal(fw.w.cpu().numpy(), O.tile_fp8(codes, scale, paired=paired))
    x = torch.randn(1, K, device=_dev()).to(torch.bfloat16)
    if paired:
        out = FK.rms_gemv(x, fw, epilogue=FK.EPI_SILU_GATE)
        g, u = (f32(m(x)) for m in mods)
        want = O.silu(g) * u
        assert O.rel_err(f32(out), want) <= 1e-2
    else:
        out = FK.rms_gemv(x, fw)
        want = torch.cat([m(x) for m in mods], dim=1)
        assert O.rel_err(f32(out), f32(want)) <= 1e-2


def test_fp8_linear_any_width():
    """in_features that is not a multiple of 16 (accepted by the reference,
    models/fp8_linear.py:47-66) runs on zero-padded rows."""
    N, K = 96, 100
    lin, w = _linear(N, K, 55, "cuda")
    mod = F8.Fp8Linear(lin)
    assert tuple(mod.weight_fp8.shape) == (N, K)
    codes, scale = O.quantize_fp8_linear(w)
    assert np.array_equal(mod.weight_fp8.view(torch.uint8).cpu().numpy(), codes)
    x = torch.randn(3, K, device=_dev()).to(torch.bfloat16)
    ref = O.gemv_ref(x.float().cpu().numpy(), O.dequant_fp8(codes, scale))
    assert O.rel_err(f32(mod(x)), ref) <= TOL
    with torch.no_grad():
        mod.weight_fp8.copy_(torch.zeros_like(mod.weight_fp8))     # the padded copy follows the buffer
    assert torch.count_nonzero(mod(x)) == 0


@pytest.mark.parametrize("kind", ["int4_tiled", "int4_rowmajor", "fp8"])
def test_modules_empty_batch(kind):
    """No tokens in, an empty output of the right shape out, with nothing
    launched -- as torch's int4 / fp8 matmuls return for an empty batch."""
    N, K = 64, 256
    lin, _ = _linear(N, K, 77, "cuda")
    if kind == "fp8":
        mod = F8.Fp8Linear(lin)
    else:
        mod = I4.Int4Linear(lin, group_size=128)
        if kind == "int4_rowmajor":
            mod = I4.Int4Linear(lin, group_size=32)   # group 32 keeps the row-major layout
    for shape in ((0, K), (2, 0, K)):
        x = torch.randn(*shape, device=_dev()).to(torch.bfloat16)
        out = mod(x)
        assert out.shape == (*shape[:-1], N) and out.dtype == x.dtype
    torch.cuda.synchronize()


def test_rmsnorm_and_silu_mul_kernels():
    M, K = 3, 2560
    _, gamma, x = O.synth(1, K, M, seed=60)
    y = FK.rmsnorm(bf16_tensor(x), bf16_tensor(gamma), 1e-6)
    ref = O.rmsnorm_f32(O.bf16_bits_to_f32(x), O.bf16_bits_to_f32(gamma))
    assert np.all(np.abs(f32(y) - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-30)
    g = torch.randn(M, 1000, device=_dev()).to(torch.bfloat16)
    u = torch.randn(M, 1000, device=_dev()).to(torch.bfloat16)
    got = f32(FK.silu_mul(g, u))
    want = O.silu(f32(g)) * f32(u)
    assert np.all(np.abs(got - want) <= 2.0 ** -7 * np.abs(want) + 1e-6)


# ---------------------------------------------------------------------------
# HIP graph capture: every replay equals the eager result
# ---------------------------------------------------------------------------


def test_graph_replays_match_eager():
    N, K, M = 2048, 2560, 1
    w, gamma, x = O.synth(N, K, M, seed=70)
    fw = FK.FusedWeight(torch.from_numpy(w).to(_dev()), bits=4)
    xd, gd = bf16_tensor(x), bf16_tensor(gamma)
    out = torch.empty(M, N // 2, device=_dev(), dtype=torch.bfloat16)
    eager = FK.rms_gemv(xd, fw, gd, 1e-6, epilogue=FK.EPI_SILU_GATE).clone()
    args = fw.gemv_args()
    wt, wf = args.pop("w"), args.pop("wfmt")
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st):
        with torch.cuda.graph(g, stream=st):
            G.gemv(xd, wt, wf, N, gamma=gd, eps=1e-6, epilogue=G.EPI_SILU_GATE, out=out, **args)
    torch.cuda.current_stream().wait_stream(st)
    for i in range(4):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        _ = (xd.float() * 2).sum().item()  # unrelated eager work between replays
