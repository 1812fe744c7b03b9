"""Quantized checkpoint save / shells / load round trip and the int4 layout
converter (CPU; the GPU forward round trip is in test_gpu_checkpoint.py).
Mirrors the flow of the reference's test_quantized_checkpoint.py minus the
model: describe -> save -> fresh skeleton -> install_shells -> load."""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch
from torch import nn

from oracle import bz_oracle as O

from breeze_amd import quantized_checkpoint as Q
from breeze_amd import fp8_linear as F8
from breeze_amd.fp8_linear import Fp8Linear
from breeze_amd.fp8_linear import tiled_shape as fp8_tiled_shape
from breeze_amd.int4_linear import LAYOUT_ROWMAJOR, LAYOUT_TILED, Int4Linear, tiled_shape


def _int4_shell(n, k, g, gen, tiled=False):
    """An Int4Linear holding random bytes: tiled [N/16, chunk/4] or row-major [N, K/8]."""
    m = Int4Linear.__new__(Int4Linear)
    nn.Module.__init__(m)
    m.in_features, m.out_features, m.group_size = k, n, g
    shape = tiled_shape(n, k) if tiled else (n, k // 8)
    m.register_buffer("weight_int4", torch.randint(-2**31, 2**31 - 1, shape, dtype=torch.int32, generator=gen))
    m.register_buffer("scales_zeros", torch.randn(k // g, n, 2, generator=gen).to(torch.bfloat16))
    return m


def _fp8_shell(n, k, gen, tiled=False):
    """An Fp8Linear holding random codes: tiled [N/16, 16 K + 128] or the
    reference's row-major [N, K]."""
    m = Fp8Linear.__new__(Fp8Linear)
    nn.Module.__init__(m)
    m.in_features, m.out_features = k, n
    shape = fp8_tiled_shape(n, k) if tiled else (n, k)
    m.register_buffer("weight_fp8", torch.randn(*shape, generator=gen).to(torch.float8_e4m3fn))
    m.register_buffer("weight_scale", torch.rand(1, n, generator=gen))
    return m


class _Block(nn.Module):
    def __init__(self):
        super().__init__()
        self.norm = nn.LayerNorm(128)
        self.mlp = nn.Module()
        self.mlp.gate_proj = nn.Linear(128, 256, bias=False)
        self.mlp.up_proj = nn.Linear(128, 256, bias=False)
        self.mlp.down_proj = nn.Linear(256, 128, bias=False)


def _quantized_block():
    """gate: tiled int4 (group 128); up: row-major int4 (group 32); down: fp8."""
    gen = torch.Generator().manual_seed(0)
    blk = _Block()
    blk.mlp.gate_proj = _int4_shell(256, 128, 128, gen, tiled=True)
    blk.mlp.up_proj = _int4_shell(256, 128, 32, gen)
    blk.mlp.down_proj = _fp8_shell(128, 256, gen)
    return blk


def test_round_trip(tmp_path):
    blk = _quantized_block()
    man = Q.save_quantized(blk, tmp_path, {"int4": "mlp"}, source="synthetic")
    assert man["modules"]["mlp.gate_proj"]["layout"] == LAYOUT_TILED == Q.INT4_LAYOUT
    assert man["modules"]["mlp.up_proj"]["layout"] == LAYOUT_ROWMAJOR
    assert man["modules"]["mlp.gate_proj"]["shapes"]["weight_int4"] == list(tiled_shape(256, 128))
    assert man["modules"]["mlp.down_proj"]["kind"] == "fp8"
    assert man["tensor_count"] == len(blk.state_dict())
    assert json.loads((tmp_path / Q.MANIFEST_NAME).read_text()) == man
    fresh = _Block()
    manifest = Q.read_manifest(tmp_path)
    assert Q.install_shells(fresh, manifest, "cpu") == 3
    stats = Q.load_quantized_state(fresh, tmp_path, "cpu")
    assert stats["missing"] == 0 and stats["unexpected"] == 0
    for (ka, va), (kb, vb) in zip(sorted(blk.state_dict().items()), sorted(fresh.state_dict().items())):
        assert ka == kb
        assert torch.equal(va.view(torch.uint8) if va.dtype == torch.float8_e4m3fn else va,
                           vb.view(torch.uint8) if vb.dtype == torch.float8_e4m3fn else vb), ka


def test_shells_on_meta_and_host_prefixes(tmp_path):
    Q.save_quantized(_quantized_block(), tmp_path, {}, source="synthetic")
    fresh = _Block()
    Q.install_shells(fresh, Q.read_manifest(tmp_path), "meta")
    assert fresh.mlp.gate_proj.weight_int4.is_meta
    stats = Q.load_quantized_state(fresh, tmp_path, "cpu", host_prefixes=("norm.",))
    assert stats["missing"] == 0
    assert not any(t.is_meta for t in list(fresh.parameters()) + list(fresh.buffers()))


def test_refuses_foreign_layouts_kinds_and_versions(tmp_path):
    Q.save_quantized(_quantized_block(), tmp_path, {}, source="synthetic")
    man = Q.read_manifest(tmp_path)
    no_tag = json.loads(json.dumps(man))
    del no_tag["modules"]["mlp.gate_proj"]["layout"]
    with pytest.raises(ValueError, match="tinygemm"):
        Q.install_shells(_Block(), no_tag, "cpu")
    int8 = json.loads(json.dumps(man))
    int8["modules"]["mlp.up_proj"]["kind"] = "int8"
    with pytest.raises(ValueError, match="not part of this build"):
        Q.install_shells(_Block(), int8, "cpu")
    unknown = json.loads(json.dumps(man))
    unknown["modules"]["mlp.gate_proj"]["layout"] = "something-else"
    with pytest.raises(ValueError, match="tinygemm"):
        Q.install_shells(_Block(), unknown, "cpu")
    man["version"] = 99
    (tmp_path / Q.MANIFEST_NAME).write_text(json.dumps(man))
    with pytest.raises(ValueError, match="unsupported checkpoint version"):
        Q.read_manifest(tmp_path)


@pytest.mark.parametrize("path,key,value", [
    ("mlp.gate_proj", "weight_int4", [256, 16]),      # a row-major shape under the tiled tag
    ("mlp.up_proj", "weight_int4", [256, 8]),         # short rows
    ("mlp.up_proj", "scales_zeros", [2, 256, 2]),     # groups of 64 recorded as 32
    ("mlp.down_proj", "weight_fp8", [128, 128]),
    ("mlp.down_proj", "weight_scale", [128]),
])
def test_refuses_manifest_shapes_that_do_not_match(tmp_path, path, key, value):
    """A manifest whose buffer shapes disagree with the module's features
    and group is refused before any buffer is made: the GEMV would read past
    a short buffer."""
    Q.save_quantized(_quantized_block(), tmp_path, {}, source="synthetic")
    man = Q.read_manifest(tmp_path)
    man["modules"][path]["shapes"][key] = value
    with pytest.raises(ValueError, match="do not match"):
        Q.install_shells(_Block(), man, "cpu")


def test_refuses_untileable_tiled_entry(tmp_path):
    Q.save_quantized(_quantized_block(), tmp_path, {}, source="synthetic")
    man = Q.read_manifest(tmp_path)
    man["modules"]["mlp.up_proj"]["layout"] = LAYOUT_TILED      # group 32 has no tiled layout
    with pytest.raises(ValueError, match="no tiled layout"):
        Q.install_shells(_Block(), man, "cpu")


def test_fp8_layout_tags(tmp_path):
    """fp8 entries carry their layout: a tiled module round-trips under
    bz-fp8-tiled16-v1; an entry without a tag (the reference's manifest) is
    its row-major [N, K] buffer; an unknown tag, or the tiled tag on a shape
    that has no tiled layout, is refused."""
    gen = torch.Generator().manual_seed(5)
    blk = _Block()
    blk.mlp.gate_proj = _fp8_shell(256, 128, gen, tiled=True)
    blk.mlp.up_proj = _fp8_shell(256, 128, gen)
    blk.mlp.down_proj = _fp8_shell(128, 256, gen, tiled=True)
    man = Q.save_quantized(blk, tmp_path, {"fp8": "mlp"}, source="synthetic")
    assert man["modules"]["mlp.gate_proj"]["layout"] == F8.LAYOUT_TILED
    assert man["modules"]["mlp.gate_proj"]["shapes"]["weight_fp8"] == [16, 16 * 128 + 128]
    assert man["modules"]["mlp.up_proj"]["layout"] == F8.LAYOUT_ROWMAJOR
    fresh = _Block()
    Q.install_shells(fresh, Q.read_manifest(tmp_path), "cpu")
    assert Q.load_quantized_state(fresh, tmp_path, "cpu")["missing"] == 0
    for name in ("gate_proj", "up_proj", "down_proj"):
        a, b = getattr(blk.mlp, name), getattr(fresh.mlp, name)
        assert torch.equal(a.weight_fp8.view(torch.uint8), b.weight_fp8.view(torch.uint8)), name
    untagged = json.loads(json.dumps(man))
    del untagged["modules"]["mlp.up_proj"]["layout"]
    other = _Block()
    Q.install_shells(other, untagged, "cpu")
    assert tuple(other.mlp.up_proj.weight_fp8.shape) == (256, 128)
    bad = json.loads(json.dumps(man))
    bad["modules"]["mlp.up_proj"]["layout"] = "fp8-something"
    with pytest.raises(ValueError, match="fp8 module stored in layout"):
        Q.install_shells(_Block(), bad, "cpu")
    bad = json.loads(json.dumps(man))
    bad["modules"]["mlp.up_proj"].update(layout=F8.LAYOUT_TILED, in_features=100)
    with pytest.raises(ValueError, match="no tiled layout"):
        Q.install_shells(_Block(), bad, "cpu")


def test_convert_logical_int4_matches_oracle_packing():
    rng = np.random.default_rng(3)
    q = rng.integers(0, 16, (48, 256), dtype=np.uint8)
    odd_low = torch.from_numpy(O.pack_nibbles_odd_low(q))
    sz = torch.randn(2, 48, 2).to(torch.bfloat16)
    w4, sz2 = Q.convert_logical_int4(odd_low, sz, 128)
    assert w4.dtype == torch.int32 and w4.shape == (48, 32)
    np.testing.assert_array_equal(w4.view(torch.uint8).numpy(), O.pack_nibbles_even_low(q))
    assert torch.equal(sz2, sz)
    assert torch.equal(Q.logical_int4(w4), odd_low)
    with pytest.raises(ValueError):
        Q.convert_logical_int4(odd_low, torch.zeros(3, 48, 2), 128)
