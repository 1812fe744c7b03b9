"""Quantized checkpoint round trip on the GPU: modules quantized here, saved,
rebuilt from the manifest into a fresh skeleton, loaded, and run -- the
outputs must be identical bit for bit; and a module built from the
reference's logical nibbles (via convert_logical_int4) against the oracle's
dequantize-then-matmul (bar 1e-2, the reference's; 4e-3 same-rounding)."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

from oracle import bz_oracle as O
from tests._util import f32

from breeze_amd import fp8_linear as F8
from breeze_amd import int4_linear as I4
from breeze_amd import quantized_checkpoint as Q

pytestmark = pytest.mark.gpu


class _MLP(nn.Module):
    def __init__(self, h=512, i=1024):
        super().__init__()
        self.gate_proj = nn.Linear(h, i, bias=False)
        self.up_proj = nn.Linear(h, i, bias=False)
        self.down_proj = nn.Linear(i, h, bias=False)

    def forward(self, x):
        return self.down_proj(torch.nn.functional.silu(self.gate_proj(x)) * self.up_proj(x))


class _Model(nn.Module):
    def __init__(self):
        super().__init__()
        self.a = _MLP()
        self.b = _MLP()

    def forward(self, x):
        return self.b(self.a(x))


def test_round_trip_forward_identical(tmp_path):
    torch.manual_seed(0)
    model = _Model().to("cuda", torch.bfloat16)
    I4.quantize_module_int4(model.a, min_bytes=0)
    F8.quantize_module_fp8(model.b, min_bytes=0)
    x = torch.randn(3, 512, device="cuda").to(torch.bfloat16)
    ref = model(x)
    man = Q.save_quantized(model, tmp_path, {"int4": "a", "fp8": "b"}, source="synthetic")
    assert len(man["modules"]) == 6
    with torch.device("meta"):
        fresh = _Model()
    Q.install_shells(fresh, Q.read_manifest(tmp_path), "meta")
    stats = Q.load_quantized_state(fresh, tmp_path, "cuda")
    assert stats["missing"] == 0 and stats["unexpected"] == 0
    assert not any(t.is_meta for t in list(fresh.parameters()) + list(fresh.buffers()))
    got = fresh(x)
    assert torch.equal(got, ref)


def test_rowmajor_checkpoint_is_retiled_on_load(tmp_path):
    """A checkpoint whose int4 modules hold the row-major layout (tag
    bz-int4-rowmajor-evenlow-v1) loads onto the GPU re-tiled: the same bytes
    as a module quantized in the tiled layout, the same outputs."""
    torch.manual_seed(1)
    model = _MLP().to("cuda", torch.bfloat16)
    I4.quantize_module_int4(model, min_bytes=0)
    x = torch.randn(2, 512, device="cuda").to(torch.bfloat16)
    ref = model(x)
    tiled = {n: getattr(model, n).weight_int4.clone() for n in ("gate_proj", "up_proj", "down_proj")}
    for name, w in tiled.items():
        mod = getattr(model, name)
        packed, _ = O.untile_int4(w.view(torch.uint8).cpu().numpy().reshape(-1), mod.out_features, mod.in_features)
        mod.weight_int4 = torch.from_numpy(packed).view(torch.int32).cuda()
    man = Q.save_quantized(model, tmp_path, {}, source="synthetic")
    assert {e["layout"] for e in man["modules"].values()} == {I4.LAYOUT_ROWMAJOR}
    fresh = _MLP()
    Q.install_shells(fresh, Q.read_manifest(tmp_path), "meta")
    Q.load_quantized_state(fresh, tmp_path, "cuda")
    for name, w in tiled.items():
        assert torch.equal(getattr(fresh, name).weight_int4, w), name
    assert torch.equal(fresh(x), ref)


def test_reference_fp8_checkpoint_is_retiled_on_load(tmp_path):
    """A checkpoint of the reference's Fp8Linear buffers -- row-major [N, K]
    codes, no layout tag in its manifest entries -- loads onto the GPU
    re-tiled: the bytes of a module quantized here, the same outputs."""
    torch.manual_seed(2)
    model = _MLP().to("cuda", torch.bfloat16)
    F8.quantize_module_fp8(model, min_bytes=0)
    x = torch.randn(2, 512, device="cuda").to(torch.bfloat16)
    ref = model(x)
    tiled = {n: getattr(model, n).weight_fp8.view(torch.uint8).clone() for n in ("gate_proj", "up_proj", "down_proj")}
    for name, w in tiled.items():
        mod = getattr(model, name)
        codes, _ = O.untile_fp8(w.cpu().numpy().reshape(-1), mod.out_features, mod.in_features)
        mod.weight_fp8 = torch.from_numpy(codes).cuda().view(torch.float8_e4m3fn)
    man = Q.save_quantized(model, tmp_path, {}, source="synthetic")
    assert {e["layout"] for e in man["modules"].values()} == {F8.LAYOUT_ROWMAJOR}
    for e in man["modules"].values():   # as the reference writes it: no layout tag
        del e["layout"]
    (tmp_path / Q.MANIFEST_NAME).write_text(__import__("json").dumps(man))
    fresh = _MLP()
    Q.install_shells(fresh, Q.read_manifest(tmp_path), "meta")
    Q.load_quantized_state(fresh, tmp_path, "cuda")
    for name, w in tiled.items():
        assert F8.layout_of(getattr(fresh, name).weight_fp8, w.shape[0] * 16, 0) == F8.LAYOUT_TILED
        assert torch.equal(getattr(fresh, name).weight_fp8.view(torch.uint8), w), name
    assert torch.equal(fresh(x), ref)
    man2 = Q.save_quantized(fresh, tmp_path / "again", {}, source="synthetic")
    assert {e["layout"] for e in man2["modules"].values()} == {F8.LAYOUT_TILED}


def test_module_from_logical_nibbles_matches_oracle():
    rng = np.random.default_rng(4)
    N, K = 512, 1024
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    q, s, lo, z = O.quantize_int4_asym(w, 128)
    sz = O.scales_zeros(s, z)
    w4, sz_t = Q.convert_logical_int4(torch.from_numpy(O.pack_nibbles_odd_low(q)),
                                      torch.from_numpy(sz.view(np.int16)).view(torch.bfloat16))
    m = I4.Int4Linear.__new__(I4.Int4Linear)
    nn.Module.__init__(m)
    m.in_features, m.out_features, m.group_size = K, N, 128
    m.register_buffer("weight_int4", w4.cuda())
    m.register_buffer("scales_zeros", sz_t.cuda())
    x = O.round_bf16(rng.standard_normal((2, K)).astype(np.float32))
    xd = torch.from_numpy(x).to("cuda", torch.bfloat16)
    ref = O.gemv_ref(x, O.dequant_int4_zp(q, sz, 128))
    assert O.rel_err(f32(m(xd).float()), ref) <= 4e-3
    assert I4.retile(m) and I4.layout_of(m.weight_int4, N, K) == I4.LAYOUT_TILED
    assert O.rel_err(f32(m(xd).float()), ref) <= 4e-3
