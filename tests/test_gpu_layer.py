"""FusedDecoderLayer and install_fused_* on the GPU against transformers'
own Qwen3 decoder layer (the reference's unfused path), run in float32 on
the CPU with the same weights -- the dequantized w_eff of the oracle's
quantizers for the int4 / fp8 variants -- and the same cache state
(models/fused/test_layer.py:21-96 is the reference's version of this check).

Bar: max|fused - ref| / max|ref| <= 1e-2 per decode step (the reference's
GEMV bar), and the caches agree to a bf16 step."""

from __future__ import annotations

import copy
import types

import numpy as np
import pytest
import torch

from oracle import bz_oracle as O

from breeze_amd import fp8_linear as F8
from breeze_amd import int4_linear as I4
from breeze_amd.fused.install import install_fused_backbone, install_fused_depth, static_cache
from breeze_amd.fused.layer import FusedDecoderLayer

pytestmark = pytest.mark.gpu

TOL = 1e-2
DEV = "cuda"


def _cfg(H=512, I=1024, HQ=8, HKV=2, D=128, layers=1):
    from transformers import Qwen3Config

    cfg = Qwen3Config(hidden_size=H, intermediate_size=I, num_attention_heads=HQ, num_key_value_heads=HKV,
                      head_dim=D, num_hidden_layers=layers, rms_norm_eps=1e-6, max_position_embeddings=4096,
                      vocab_size=64)
    cfg._attn_implementation = "eager"
    return cfg


def _layer(cfg, seed=0):
    from transformers.models.qwen3.modeling_qwen3 import Qwen3DecoderLayer

    torch.manual_seed(seed)
    layer = Qwen3DecoderLayer(cfg, layer_idx=0).float().eval()
    with torch.no_grad():
        for p in layer.parameters():
            if p.dim() == 2:
                p.normal_(0, 0.03)
        for n in ("input_layernorm", "post_attention_layernorm"):
            getattr(layer, n).weight.normal_(1, 0.1)
        layer.self_attn.q_norm.weight.normal_(1, 0.1)
        layer.self_attn.k_norm.weight.normal_(1, 0.1)
        for p in layer.parameters():   # bf16-representable, so both sides hold the same weights
            p.copy_(p.to(torch.bfloat16).float())
    return layer


def _dequant_oracle(layer, variant):
    """CPU copy whose MLP weights are the oracle's w_eff for the variant."""
    ref = copy.deepcopy(layer)
    for n in ("gate_proj", "up_proj", "down_proj"):
        lin = getattr(ref.mlp, n)
        w = lin.weight.detach().numpy().astype(np.float32)
        if variant == "int4":
            q, s, lo, z = O.quantize_int4_asym(w, 128)
            w_eff = O.dequant_int4_zp(q, O.scales_zeros(s, z), 128)
        else:
            codes, scale = O.quantize_fp8_linear(w)
            w_eff = O.dequant_fp8(codes, scale)
        with torch.no_grad():
            lin.weight.copy_(torch.from_numpy(np.asarray(w_eff, np.float32)))
    return ref


def _fused(layer, variant, attn_bits=16):
    g = copy.deepcopy(layer).to(DEV, torch.bfloat16)
    if variant == "int4":
        st = I4.quantize_module_int4(g, min_bytes=0)
        assert st["converted"] == 3
    elif variant == "fp8":
        st = F8.quantize_module_fp8(g, min_bytes=0)
        assert st["converted"] == 3
    return FusedDecoderLayer(g, 0, attn_bits=attn_bits)


def _run_steps(cfg, ref, fused, B, S, steps, pass_position=True, seed=1):
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding

    rot_cpu = Qwen3RotaryEmbedding(cfg)
    rot_gpu = Qwen3RotaryEmbedding(cfg).to(DEV)
    c_ref = static_cache(cfg, S, B)
    c_fus = static_cache(cfg, S, B)
    mask = torch.full((B, 1, 1, S), torch.finfo(torch.float32).min)
    g = torch.Generator().manual_seed(seed)
    errs = []
    for t in range(steps):
        x = torch.randn(B, 1, cfg.hidden_size, generator=g).to(torch.bfloat16).float()
        pid = torch.full((B, 1), t)
        mask[:, :, :, t] = 0.0
        if t == 3 and B > 1:
            mask[1, :, :, 1] = torch.finfo(torch.float32).min   # row 1: position 1 becomes padding
        with torch.no_grad():
            y = ref(x, attention_mask=mask, position_ids=pid, past_key_values=c_ref, use_cache=True,
                    position_embeddings=rot_cpu(x, pid))
            xg = x.to(DEV, torch.bfloat16)
            pe = rot_gpu(xg, pid.to(DEV))
            kw = {"cache_position": torch.tensor([t], device=DEV)} if pass_position else {}
            o = fused(xg, attention_mask=mask.to(DEV, torch.bfloat16), position_ids=pid.to(DEV),
                      past_key_values=c_fus, use_cache=True, position_embeddings=pe, **kw)
        y = y[0] if isinstance(y, tuple) else y
        errs.append(O.rel_err(o.float().cpu().numpy(), y.numpy()))
    return errs, c_ref, c_fus


@pytest.mark.parametrize("variant,attn_bits", [("bf16", 16), ("bf16", 8), ("int4", 16), ("fp8", 8)])
def test_fused_layer_matches_qwen3(variant, attn_bits):
    cfg = _cfg()
    layer = _layer(cfg)
    ref = layer if variant == "bf16" else _dequant_oracle(layer, variant)
    if attn_bits == 8:   # the fused path quantizes the attention projections: give the reference the same
        ref = copy.deepcopy(ref)
        for n in ("q_proj", "k_proj", "v_proj", "o_proj"):
            lin = getattr(ref.self_attn, n)
            codes, scale = O.pack_fp8(lin.weight.detach().numpy())
            with torch.no_grad():
                lin.weight.copy_(torch.from_numpy(np.asarray(O.dequant_fp8(codes, scale), np.float32)))
    fused = _fused(layer, variant, attn_bits)
    errs, c_ref, c_fus = _run_steps(cfg, ref, fused, B=2, S=64, steps=12)
    assert max(errs) <= TOL, errs
    k_ref, k_fus = c_ref.layers[0].keys.numpy(), c_fus.layers[0].keys.float().cpu().numpy()
    assert O.rel_err(k_fus, k_ref) <= TOL
    assert O.rel_err(c_fus.layers[0].values.float().cpu().numpy(), c_ref.layers[0].values.numpy()) <= TOL


def test_fused_layer_real_head_shape_long_cache():
    """The backbone's head shape (16 q / 4 kv heads of 256) on a cache of 512
    positions: splits > 1 and positions past the first split."""
    cfg = _cfg(H=1024, I=1024, HQ=16, HKV=4, D=256)
    layer = _layer(cfg, seed=3)
    fused = _fused(layer, "bf16")
    errs, _, _ = _run_steps(cfg, layer, fused, B=2, S=512, steps=6)
    assert max(errs) <= TOL, errs


def test_fused_layer_without_cache_position_uses_the_cache_counter():
    """transformers >= 5 passes no cache_position: the step position comes
    from the cache's fill counter, which the fused step advances."""
    cfg = _cfg()
    layer = _layer(cfg, seed=4)
    fused = _fused(layer, "bf16")
    errs, _, c_fus = _run_steps(cfg, layer, fused, B=2, S=32, steps=5, pass_position=False)
    assert max(errs) <= TOL, errs
    counter = getattr(c_fus.layers[0], "cumulative_length", None)
    if isinstance(counter, torch.Tensor):
        assert int(counter) == 5


def test_fused_layer_short_prefill_t2():
    """The depth decoder's 2-position start: one call with T = 2 equals two
    decode steps (models/fused/layer.py:69-79)."""
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding

    cfg = _cfg()
    layer = _layer(cfg, seed=5)
    fused = _fused(layer, "bf16")
    B, S = 2, 18
    c_ref, c_fus = static_cache(cfg, S, B), static_cache(cfg, S, B)
    x2 = torch.randn(B, 2, cfg.hidden_size).to(torch.bfloat16).float()
    pid = torch.arange(2).unsqueeze(0).expand(B, 2)
    m2 = torch.full((B, 1, 2, S), torch.finfo(torch.float32).min)
    m2[:, :, 0, :1] = 0
    m2[:, :, 1, :2] = 0
    with torch.no_grad():
        r2 = layer(x2, attention_mask=m2, position_ids=pid, past_key_values=c_ref, use_cache=True,
                   position_embeddings=Qwen3RotaryEmbedding(cfg)(x2, pid))
        xg = x2.to(DEV, torch.bfloat16)
        o2 = fused(xg, attention_mask=m2.to(DEV, torch.bfloat16), position_ids=pid.to(DEV), past_key_values=c_fus,
                   use_cache=True, cache_position=torch.arange(2, device=DEV),
                   position_embeddings=Qwen3RotaryEmbedding(cfg).to(DEV)(xg, pid.to(DEV)))
    r2 = r2[0] if isinstance(r2, tuple) else r2
    assert o2.shape == (B, 2, cfg.hidden_size)
    assert O.rel_err(o2.float().cpu().numpy(), r2.numpy()) <= TOL


def test_fused_layer_falls_back_without_cache():
    """No cache (or no mask, or T > 4): the original layer runs.  It is kept
    in float32 here, so its attention matmuls are float32 ones."""
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding

    cfg = _cfg()
    layer = _layer(cfg, seed=6)
    fused = FusedDecoderLayer(copy.deepcopy(layer).to(DEV), 0)
    called = []
    fused.orig.register_forward_hook(lambda *a: called.append(1))
    x = torch.randn(2, 5, cfg.hidden_size, device=DEV)
    pid = torch.arange(5, device=DEV).unsqueeze(0).expand(2, 5)
    pe = Qwen3RotaryEmbedding(cfg).to(DEV)(x, pid)
    with torch.no_grad():
        y = fused(x, attention_mask=None, position_ids=pid, past_key_values=None, position_embeddings=pe)
        r = layer(x.cpu(), attention_mask=None, position_ids=pid.cpu(), past_key_values=None,
                  position_embeddings=tuple(t.cpu() for t in pe))
    assert called
    y = y[0] if isinstance(y, tuple) else y
    r = r[0] if isinstance(r, tuple) else r
    assert O.rel_err(y.cpu().numpy(), r.numpy()) <= 1e-4


def _forbid_unfused(model_layers):
    """Raise before an unfused bf16 layer would run its attention on the GPU."""
    def stop(mod, args, kwargs):
        raise AssertionError("the unfused layer was called")

    for layer in model_layers:
        layer.orig.register_forward_pre_hook(stop, with_kwargs=True)


def _model(cfg, seed):
    from transformers.models.qwen3.modeling_qwen3 import Qwen3Model

    torch.manual_seed(seed)
    m = Qwen3Model(cfg).float().eval()
    with torch.no_grad():
        for p in m.parameters():
            if p.dim() == 2:
                p.normal_(0, 0.03)
            else:
                p.normal_(1, 0.1)
            p.copy_(p.to(torch.bfloat16).float())
    return m


def test_install_fused_backbone_runs_a_whole_model():
    """install_fused_backbone on a 3-layer Qwen3 backbone; the model's own
    forward (transformers masks, rotary, no cache_position) for a 3-token
    start then single-token steps, against the CPU float32 model."""
    cfg = _cfg(layers=3)
    ref = _model(cfg, 7)
    gpu = copy.deepcopy(ref).to(DEV, torch.bfloat16)
    model = types.SimpleNamespace(backbone_model=gpu)
    assert install_fused_backbone(model, batch_size=2, max_seq_len=64) == 3
    assert install_fused_backbone(model, batch_size=2, max_seq_len=64) == 0   # idempotent
    assert all(isinstance(layer, FusedDecoderLayer) for layer in gpu.layers)
    _forbid_unfused(gpu.layers)
    B, S = 2, 64
    c_ref, c_gpu = static_cache(cfg, S, B), static_cache(cfg, S, B)
    g = torch.Generator().manual_seed(8)
    for t, n in enumerate([3, 1, 1, 1, 1]):
        x = torch.randn(B, n, cfg.hidden_size, generator=g).to(torch.bfloat16).float()
        with torch.no_grad():
            r = ref(inputs_embeds=x, past_key_values=c_ref, use_cache=True).last_hidden_state
            o = gpu(inputs_embeds=x.to(DEV, torch.bfloat16), past_key_values=c_gpu, use_cache=True).last_hidden_state
        assert O.rel_err(o.float().cpu().numpy(), r.numpy()) <= TOL, t


def test_install_fused_depth():
    cfg = _cfg(layers=2)
    cfg.num_codebooks = 15
    ref = _model(cfg, 9)
    gpu = copy.deepcopy(ref).to(DEV, torch.bfloat16)
    model = types.SimpleNamespace(depth_decoder=types.SimpleNamespace(model=gpu))
    assert install_fused_depth(model, batch_size=2) == 2
    assert all(isinstance(layer, FusedDecoderLayer) for layer in gpu.layers)
