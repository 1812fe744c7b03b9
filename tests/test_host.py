"""Host-side logic of the reference-shaped modules, CPU only: constructor
rejections and their messages (models/int4_linear.py:78-79,90-93,
models/fp8_linear.py:49-50), the quantize_module_* swap policy and stats
dicts (models/int4_linear.py:118-164, models/fp8_linear.py:89-122), the
FusedWeight plumbing and the Python wrapper's own argument checks.  Nothing
here launches a kernel."""

from __future__ import annotations

import pytest
import torch
from torch import nn

from breeze_amd import fp8_linear as F8
from breeze_amd import gemv as G
from breeze_amd import int4_linear as I4
from breeze_amd.fused import kernels as FK


def test_reference_constants():
    assert I4.GROUP_SIZE == 128
    assert I4.MIN_QUANT_BYTES == F8.MIN_QUANT_BYTES == 8 * 1024 * 1024
    assert I4.DEFAULT_TARGET_NAMES == F8.DEFAULT_TARGET_NAMES == ("gate_proj", "up_proj", "down_proj")
    assert F8.FP8_MAX == 448.0 and F8.FP8_DTYPE is torch.float8_e4m3fn
    assert FK.GROUP == 128


def test_int4_rejects_bias():
    with pytest.raises(ValueError, match="Int4Linear expects a bias-free Linear"):
        I4.Int4Linear(nn.Linear(256, 16, bias=True))


def test_int4_rejects_group_mismatch():
    with pytest.raises(ValueError, match="in_features 200 not divisible by group 128"):
        I4.Int4Linear(nn.Linear(200, 16, bias=False))
    with pytest.raises(ValueError, match="power of two"):
        I4.Int4Linear(nn.Linear(288, 16, bias=False), group_size=96)


def test_fp8_rejects_bias():
    # any in_features is accepted (models/fp8_linear.py:47-66); only a bias is refused
    with pytest.raises(ValueError, match="Fp8Linear expects a bias-free Linear"):
        F8.Fp8Linear(nn.Linear(256, 16, bias=True))


class _Mlp(nn.Module):
    def __init__(self, k, n, bias=False):
        super().__init__()
        self.gate_proj = nn.Linear(k, n, bias=bias)
        self.up_proj = nn.Linear(k, n, bias=bias)
        self.down_proj = nn.Linear(n, k, bias=bias)
        self.other = nn.Linear(k, n, bias=False)


class _Model(nn.Module):
    def __init__(self):
        super().__init__()
        self.layers = nn.ModuleList([_Mlp(64, 96) for _ in range(3)])
        self.biased = _Mlp(64, 96, bias=True)


def test_quantize_module_int4_policy_small_layers():
    m = _Model()
    before = {n: id(c) for n, c in m.named_modules()}
    stats = I4.quantize_module_int4(m)  # every target is below 8 MB
    assert stats == {"converted": 0, "skipped_below_threshold": 9, "skipped_unsupported": 0,
                     "weight_bytes_saved": 0}
    assert {n: id(c) for n, c in m.named_modules()} == before


def test_quantize_module_int4_unsupported_kept():
    m = _Model()
    # threshold 0: every target is attempted; no width (64, 96) is a multiple
    # of the group, so each constructor rejects its layer before quantizing
    stats = I4.quantize_module_int4(m, min_bytes=0, group_size=128)
    assert stats["converted"] == 0
    assert stats["skipped_unsupported"] == 9 and stats["skipped_below_threshold"] == 0
    assert all(type(l.gate_proj) is nn.Linear for l in m.layers)


def test_quantize_module_target_names():
    m = _Model()
    stats = I4.quantize_module_int4(m, target_names=("other",))
    assert stats["skipped_below_threshold"] == 4    # the four bias-free 'other' layers
    stats = I4.quantize_module_int4(m, target_names=())
    assert stats["skipped_below_threshold"] == 13   # empty targets: every bias-free Linear


def test_quantize_module_fp8_small_layers():
    m = _Model()
    stats = F8.quantize_module_fp8(m)
    assert stats == {"converted": 0, "skipped_below_threshold": 9, "weight_bytes_saved": 0}


def test_quantize_module_fp8_errors_propagate(monkeypatch):
    """quantize_module_fp8 lets a construction error escape (the reference
    builds Fp8Linear unguarded, models/fp8_linear.py:113)."""
    class Mlp(nn.Module):
        def __init__(self):
            super().__init__()
            self.gate_proj = nn.Linear(96, 8, bias=False)

    def refuse(weight, amax_floor):
        raise ValueError("refused")

    monkeypatch.setattr(F8, "quantize_fp8_device", refuse)
    with pytest.raises(ValueError, match="refused"):
        F8.quantize_module_fp8(Mlp(), min_bytes=0)


def test_fused_weight_plumbing():
    fw = FK.FusedWeight.__new__(FK.FusedWeight)
    fw.bits, fw.N, fw.K, fw.group, fw.layout = 4, 32, 256, 128, "zp"
    fw.w = torch.zeros(32, 128, dtype=torch.uint8)
    fw.s = torch.zeros(2, 32, 2, dtype=torch.bfloat16)
    fw.z = None
    a = fw.gemv_args()
    assert a["wfmt"] == G.W_INT4_ZP and a["group"] == 128 and a["sc0"] is fw.s
    assert fw.nbytes() == 32 * 128 + 2 * 32 * 2 * 2
    fw.layout, fw.z = "min", torch.zeros(32, 2, dtype=torch.bfloat16)
    fw.s = torch.zeros(32, 2, dtype=torch.bfloat16)
    a = fw.gemv_args()
    assert a["wfmt"] == G.W_INT4_MIN and a["sc1"] is fw.z
    fw.bits, fw.s, fw.z = 8, torch.ones(32), None
    fw.w = torch.zeros(32, 256, dtype=torch.float8_e4m3fn)
    a = fw.gemv_args()
    assert a["wfmt"] == G.W_FP8 and a["w"].dtype == torch.uint8
    fw.bits, fw.s, fw.layout = 16, None, "bf16"
    assert FK.FusedWeight.gemv_args(fw)["wfmt"] == G.W_BF16
    fw.w = torch.zeros(2, 1024, dtype=torch.uint8)
    for bits, layout, wfmt in ((4, "tiled", G.W_INT4_TILED), (4, "tiled-paired", G.W_INT4_TILED_PAIRED),
                               (8, "tiled", G.W_FP8_TILED), (8, "tiled-paired", G.W_FP8_TILED_PAIRED)):
        fw.bits, fw.layout = bits, layout
        a = fw.gemv_args()
        assert a["wfmt"] == wfmt and a["w"] is fw.w and "sc0" not in a
    assert fw.nbytes() == 2048
    c = fw.clone()
    assert c.layout == fw.layout and c.w is not fw.w and torch.equal(c.w, fw.w)


class _Lin:
    def __init__(self, n, k):
        self.out_features, self.in_features = n, k


def test_stack_shape_rules():
    assert FK._stack_shape([_Lin(64, 256), _Lin(32, 256)], False) == (96, 256)
    assert FK._stack_shape([_Lin(64, 256), _Lin(64, 256)], True) == (128, 256)
    with pytest.raises(ValueError, match="different in_features"):
        FK._stack_shape([_Lin(64, 256), _Lin(64, 128)], False)
    with pytest.raises(ValueError, match="paired"):
        FK._stack_shape([_Lin(64, 256), _Lin(32, 256)], True)
    with pytest.raises(ValueError, match="paired"):
        FK._stack_shape([_Lin(64, 256)] * 3, True)


def test_int4_layout_rules():
    assert I4.tileable(2560, 10240, 128) and not I4.tileable(2560, 10240, 64)
    assert not I4.tileable(24, 256, 128) and not I4.tileable(32, 192, 128)
    rowmajor = torch.zeros(32, 256 // 8, dtype=torch.int32)
    assert I4.layout_of(rowmajor, 32, 256) == I4.LAYOUT_ROWMAJOR
    assert I4.layout_of(torch.zeros(2, 2 * 1024 // 4 + 32, dtype=torch.int32), 32, 256) == I4.LAYOUT_TILED


def test_fused_weight_rejects_bits():
    with pytest.raises(ValueError):
        FK.FusedWeight(torch.zeros(8, 128), bits=3)


def test_gemv_wrapper_checks_before_launch():
    x = torch.zeros(1, 1, 256, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="2-D"):
        G.gemv(x, torch.zeros(8, 128, dtype=torch.uint8), G.W_INT4_ZP, 8)
    with pytest.raises((RuntimeError, ValueError), match="GPU|cuda|device"):
        G.gemv(x[0], torch.zeros(8, 128, dtype=torch.uint8), G.W_INT4_ZP, 8)


def test_layout_tag():
    assert I4.LAYOUT.startswith("bz-int4-")


def test_extra_repr_strings():
    lin = I4.Int4Linear.__new__(I4.Int4Linear)
    nn.Module.__init__(lin)
    lin.in_features, lin.out_features, lin.group_size = 2560, 10240, 128
    assert lin.extra_repr() == "in_features=2560, out_features=10240, int4=True, group=128"
    f = F8.Fp8Linear.__new__(F8.Fp8Linear)
    nn.Module.__init__(f)
    f.in_features, f.out_features = 2560, 4096
    assert f.extra_repr() == "in_features=2560, out_features=4096, fp8=True"
