"""The synthetic decode step of the int4 decoder at its real shape, on the GPU,
against the oracle's dequantize-then-matmul chain.

Hidden 2560, 16 query heads x 256, 4 KV heads, MLP 10240, int4 group-128
symmetric weights; each layer is RMSNorm -> QKV GEMV (N 6144), the attention
stand-in (the query part [M, 4096] copied), o_proj K4096 + residual,
RMSNorm -> gate|up GEMV (N 2 x 10240) with SiLU-gate, down K10240 +
residual; the step ends with RMSNorm -> bf16 head K2560 N8192.  Three full
layers run here (the 26 of the timed step repeat the same launches), at
M = 1 and M = 2, in both weight layouts: the tiled decode layout (the copy
done by the QKV launch's second store, exactly as bench.py times it) and the
row-major one.  The oracle rounds every intermediate to bf16 where the GPU
path stores bf16 and computes each GEMV in float64 over W_eff; the bar on
the logits is the stated max|out - ref| / max|ref| <= 1e-2, the comparison
the reference makes between its fused and unfused layers
(models/fused/test_layer.py:53-95)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import bz_oracle as O
from tests._util import bf16_tensor, f32, u8_tensor

from breeze_amd import gemv as G

pytestmark = pytest.mark.gpu

H, QKV, ATT, MLP, VOCAB = 2560, 6144, 4096, 10240, 8192
LAYERS = 3
TOL = 1e-2

_STEP: dict = {}


def _int4(n, k, rng):
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    q, s, z = O.quantize_int4_sym(w, 128)
    sz = O.scales_zeros(s, z)
    return {"packed": O.pack_nibbles_even_low(q), "sz": sz, "w_eff": O.dequant_int4_zp(q, sz, 128)}


def _gamma(k, rng):
    return O.f32_to_bf16_bits(np.float32(1.0) + rng.standard_normal(k, dtype=np.float32) * np.float32(0.1))


def _model():
    """Oracle-quantized weights of LAYERS layers and the head (built once)."""
    if not _STEP:
        rng = np.random.default_rng(2560)
        layers = []
        for _ in range(LAYERS):
            layers.append({"qkv": _int4(QKV, H, rng), "o": _int4(H, ATT, rng), "gu": _int4(2 * MLP, H, rng),
                           "dn": _int4(H, MLP, rng), "g1": _gamma(H, rng), "g2": _gamma(H, rng)})
        head = O.f32_to_bf16_bits(rng.standard_normal((VOCAB, H), dtype=np.float32) * np.float32(0.02))
        _STEP.update(layers=layers, head=head, gf=_gamma(H, rng),
                     h0=O.f32_to_bf16_bits(rng.standard_normal((2, H), dtype=np.float32)))
    return _STEP


_ORACLE: dict = {}


def _oracle_logits(m):
    if m not in _ORACLE:
        _ORACLE[m] = _oracle_chain(m)
    return _ORACLE[m]


def _oracle_chain(m):
    st = _model()
    h = O.bf16_bits_to_f32(st["h0"][:m])
    for L in st["layers"]:
        xn = O.rmsnorm_f32(h, O.bf16_bits_to_f32(L["g1"]))
        qkv = O.round_bf16(O.gemv_ref(xn, L["qkv"]["w_eff"]).astype(np.float32))
        att = qkv[:, :ATT]
        h = O.round_bf16(O.gemv_ref(att, L["o"]["w_eff"], O.EPI_RES, h).astype(np.float32))
        xn = O.rmsnorm_f32(h, O.bf16_bits_to_f32(L["g2"]))
        mid = O.round_bf16(O.gemv_ref(xn, L["gu"]["w_eff"], O.EPI_SILU).astype(np.float32))
        h = O.round_bf16(O.gemv_ref(mid, L["dn"]["w_eff"], O.EPI_RES, h).astype(np.float32))
    xn = O.rmsnorm_f32(h, O.bf16_bits_to_f32(st["gf"]))
    return O.gemv_ref(xn, O.bf16_bits_to_f32(st["head"]))


def _device_weight(wq, k, layout, paired=False):
    packed, sz = u8_tensor(wq["packed"]), bf16_tensor(wq["sz"])
    if layout == "rowmajor":
        return {"w": packed, "wfmt": G.W_INT4_ZP, "sc0": sz, "group": 128}
    wfmt = G.W_INT4_TILED_PAIRED if paired else G.W_INT4_TILED
    return {"w": G.pack_tiled(G.W_INT4_ZP, packed, k, wfmt, sc0=sz), "wfmt": wfmt}


def _gpu_logits(m, layout):
    st = _model()
    dev = torch.device("cuda", 0)
    layers = [{"qkv": _device_weight(L["qkv"], H, layout), "o": _device_weight(L["o"], ATT, layout),
               "gu": _device_weight(L["gu"], H, layout, paired=True), "dn": _device_weight(L["dn"], MLP, layout),
               "g1": bf16_tensor(L["g1"]), "g2": bf16_tensor(L["g2"])} for L in st["layers"]]
    head, gf = bf16_tensor(st["head"]), bf16_tensor(st["gf"])
    h0 = bf16_tensor(st["h0"][:m])
    hs = torch.empty_like(h0)
    qkv = torch.empty(m, QKV, device=dev, dtype=torch.bfloat16)
    att = torch.empty(m, ATT, device=dev, dtype=torch.bfloat16)
    mid = torch.empty(m, MLP, device=dev, dtype=torch.bfloat16)
    tiled = layout == "tiled"
    for i, L in enumerate(layers):
        x_in = h0 if i == 0 else hs
        if tiled:   # the attention stand-in's copy as the QKV launch's second store
            G.gemv(x_in, n=QKV, gamma=L["g1"], out=qkv, out2=att, **L["qkv"])
        else:
            G.gemv(x_in, n=QKV, gamma=L["g1"], out=qkv, **L["qkv"])
            att.copy_(qkv[:, :ATT])
        G.gemv(att, n=H, epilogue=G.EPI_RESIDUAL, residual=x_in, out=hs, **L["o"])
        G.gemv(hs, n=2 * MLP, gamma=L["g2"], epilogue=G.EPI_SILU_GATE, out=mid, **L["gu"])
        G.gemv(mid, n=H, epilogue=G.EPI_RESIDUAL, residual=hs, out=hs, **L["dn"])
    logits = G.gemv(hs, head, G.W_BF16, VOCAB, gamma=gf)
    torch.cuda.synchronize()
    return f32(logits)


@pytest.mark.parametrize("layout", ["tiled", "rowmajor"])
@pytest.mark.parametrize("m", [1, 2])
def test_c5_step_logits_match_oracle(m, layout):
    got = _gpu_logits(m, layout)
    ref = _oracle_logits(m)
    assert got.shape == (m, VOCAB)
    err = O.rel_err(got, ref)
    assert err <= TOL, err
