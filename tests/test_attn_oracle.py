"""Pins of the attention / decoder-layer oracle (CPU only).

The oracle is checked against transformers' own Qwen3 decoder layer -- the
reference's unfused path (eager attention, StaticCache) -- in float32 on the
CPU, and against closed forms that a dropped term, a wrong sign or a wrong
head mapping would break."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import bz_attn_oracle as A
from oracle import bz_oracle as O


def _rng(seed):
    return np.random.default_rng(seed)


# ---- rope -------------------------------------------------------------------


def test_rope_identity_and_rotation():
    rng = _rng(0)
    v = rng.standard_normal((3, 5, 64))
    np.testing.assert_allclose(A.rope(v, 1.0, 0.0), v, rtol=0, atol=0)
    np.testing.assert_allclose(A.rotate_half(A.rotate_half(v)), -v, rtol=0, atol=0)
    theta = rng.uniform(-3, 3, 32)
    cos = np.concatenate([np.cos(theta)] * 2)
    sin = np.concatenate([np.sin(theta)] * 2)
    r = A.rope(v, cos, sin)
    pair = lambda a: a[..., :32] ** 2 + a[..., 32:] ** 2  # noqa: E731
    np.testing.assert_allclose(pair(r), pair(v), rtol=1e-12)
    # a quarter turn maps (x1, x2) -> (-x2, x1)
    q = A.rope(v, np.zeros(64), np.ones(64))
    np.testing.assert_allclose(q[..., :32], -v[..., 32:])
    np.testing.assert_allclose(q[..., 32:], v[..., :32])


def test_rms_head_closed_form():
    v = np.full((2, 8), 3.0)
    np.testing.assert_allclose(A.rms_head(v, np.arange(8.0), 0.0), np.tile(np.arange(8.0), (2, 1)))
    rng = _rng(1)
    x = rng.standard_normal((4, 64))
    np.testing.assert_allclose(A.rms_head(5 * x, np.ones(64), 0.0), A.rms_head(x, np.ones(64), 0.0), rtol=1e-12)


# ---- attention closed forms ----------------------------------------------------


def _cache(B, HKV, S, D, seed):
    rng = _rng(seed)
    return rng.standard_normal((B, HKV, S, D)), rng.standard_normal((B, HKV, S, D))


def test_single_position_returns_value():
    k, v = _cache(2, 2, 8, 64, 2)
    q = _rng(3).standard_normal((2, 4, 64))
    out = A.attn_decode(q, k, v, np.zeros((2, 8)), 0).reshape(2, 4, 64)
    for h in range(4):
        np.testing.assert_allclose(out[:, h], v[:, h // 2, 0], rtol=1e-12)


def test_equal_keys_give_mean_of_values():
    k, v = _cache(1, 1, 16, 64, 4)
    k[:] = k[:, :, :1]
    q = _rng(5).standard_normal((1, 3, 64))
    out = A.attn_decode(q, k, v, np.zeros((1, 16)), 9).reshape(1, 3, 64)
    np.testing.assert_allclose(out[0], np.tile(v[0, 0, :10].mean(0), (3, 1)), rtol=1e-10)


def test_mask_drops_positions_and_shift_invariance():
    k, v = _cache(1, 2, 12, 64, 6)
    q = _rng(7).standard_normal((1, 2, 64))
    m = np.zeros((1, 12))
    m[0, [1, 4]] = A.NEG_BIG
    got = A.attn_decode(q, k, v, m, 7)
    keep = [0, 2, 3, 5, 6, 7]
    ref = A.attn_decode(q, k[:, :, keep], v[:, :, keep], np.zeros((1, 6)), 5)
    np.testing.assert_allclose(got, ref, rtol=1e-10)
    np.testing.assert_allclose(A.attn_decode(q, k, v, m + 17.0, 7), got, rtol=1e-10)


def test_attention_brute_force_and_gqa_mapping():
    B, HQ, HKV, D, S, pos = 1, 4, 2, 4, 5, 3
    k, v = _cache(B, HKV, S, D, 8)
    q = _rng(9).standard_normal((B, HQ, D))
    out = A.attn_decode(q, k, v, np.zeros((B, S)), pos).reshape(B, HQ, D)
    for h in range(HQ):
        j = h // (HQ // HKV)
        s = [sum(q[0, h, d] * k[0, j, t, d] for d in range(D)) / np.sqrt(D) for t in range(pos + 1)]
        e = [np.exp(x - max(s)) for x in s]
        ref = [sum(e[t] * v[0, j, t, d] for t in range(pos + 1)) / sum(e) for d in range(D)]
        np.testing.assert_allclose(out[0, h], ref, rtol=1e-12)
    # heads 0, 1 read kv head 0 and heads 2, 3 kv head 1: swapping kv heads swaps outputs
    out2 = A.attn_decode(q[:, [2, 3, 0, 1]], k[:, ::-1], v[:, ::-1], np.zeros((B, S)), pos).reshape(B, HQ, D)
    np.testing.assert_allclose(out2, out[:, [2, 3, 0, 1]], rtol=1e-12)


@pytest.mark.parametrize("split", [1, 2, 3, 7, 8, 16])
@pytest.mark.parametrize("pos", [0, 4, 30])
def test_split_combine_equals_unsplit(split, pos):
    k, v = _cache(2, 2, 32, 64, 10)
    q = _rng(11).standard_normal((2, 4, 64)) * 3
    m = np.where(_rng(12).random((2, 32)) < 0.2, A.NEG_BIG, 0.0)
    m[:, 0] = 0.0
    np.testing.assert_allclose(A.attn_decode_split(q, k, v, m, pos, split), A.attn_decode(q, k, v, m, pos),
                               rtol=1e-10, atol=1e-12)


def test_additive_mask_conversion():
    b = np.array([[[[True, False, True, True]]]])
    np.testing.assert_array_equal(A.additive_mask(b, 3), [[0.0, A.NEG_BIG, 0.0]])
    f = np.array([[[[0.0, -5.0, 1.0, 2.0]]]], np.float32)
    np.testing.assert_array_equal(A.additive_mask(f, 4), [[0.0, -5.0, 1.0, 2.0]])


def test_qkv_rope_cache_writes_only_pos():
    B, HQ, HKV, D, S = 2, 4, 2, 64, 6
    rng = _rng(13)
    qkv = rng.standard_normal((B, (HQ + 2 * HKV) * D))
    keys, values = np.zeros((B, HKV, S, D), np.float32), np.zeros((B, HKV, S, D), np.float32)
    A.qkv_rope_cache(qkv, HQ, HKV, D, np.ones(D), np.zeros(D), 3, keys, values, cache_bf16=False)
    assert not keys[:, :, [0, 1, 2, 4, 5]].any() and not values[:, :, [0, 1, 2, 4, 5]].any()
    np.testing.assert_allclose(values[:, :, 3], qkv[:, (HQ + HKV) * D:].reshape(B, HKV, D), rtol=1e-6)
    np.testing.assert_allclose(keys[:, :, 3], qkv[:, HQ * D:(HQ + HKV) * D].reshape(B, HKV, D), rtol=1e-6)
    before = keys.copy()
    A.qkv_rope_cache(qkv, HQ, HKV, D, np.ones(D), np.zeros(D), S, keys, values)   # outside the cache
    np.testing.assert_array_equal(keys, before)


# ---- against transformers' Qwen3 decoder layer (CPU, float32) ------------------


def _hf_layer(H=256, I=384, HQ=8, HKV=2, D=64, seed=0):
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3DecoderLayer, Qwen3RotaryEmbedding

    cfg = Qwen3Config(hidden_size=H, intermediate_size=I, num_attention_heads=HQ, num_key_value_heads=HKV,
                      head_dim=D, num_hidden_layers=1, rms_norm_eps=1e-6, max_position_embeddings=512)
    cfg._attn_implementation = "eager"
    torch.manual_seed(seed)
    layer = Qwen3DecoderLayer(cfg, layer_idx=0).float().eval()
    with torch.no_grad():
        for n in ("input_layernorm", "post_attention_layernorm"):
            getattr(layer, n).weight.copy_(1 + 0.1 * torch.randn(H))
        layer.self_attn.q_norm.weight.copy_(1 + 0.1 * torch.randn(D))
        layer.self_attn.k_norm.weight.copy_(1 + 0.1 * torch.randn(D))
    return cfg, layer, Qwen3RotaryEmbedding(cfg)


def _oracle_weights(layer, HQ, HKV, D):
    a, m = layer.self_attn, layer.mlp
    f = lambda t: t.detach().float().numpy()  # noqa: E731
    return {
        "HQ": HQ, "HKV": HKV, "D": D,
        "ln1": f(layer.input_layernorm.weight), "ln2": f(layer.post_attention_layernorm.weight),
        "qn": f(a.q_norm.weight), "kn": f(a.k_norm.weight),
        "wqkv": np.concatenate([f(a.q_proj.weight), f(a.k_proj.weight), f(a.v_proj.weight)], 0),
        "wo": f(a.o_proj.weight),
        "wgu": np.concatenate([f(m.gate_proj.weight), f(m.up_proj.weight)], 0),
        "wd": f(m.down_proj.weight),
    }


def test_decoder_layer_step_matches_transformers_qwen3():
    from transformers import StaticCache

    H, HQ, HKV, D, S, B, steps = 256, 8, 2, 64, 16, 2, 7
    cfg, layer, rot = _hf_layer(H=H, HQ=HQ, HKV=HKV, D=D)
    w = _oracle_weights(layer, HQ, HKV, D)
    cache = StaticCache(config=cfg, max_cache_len=S)
    keys = np.zeros((B, HKV, S, D), np.float32)
    values = np.zeros((B, HKV, S, D), np.float32)
    mask = torch.full((B, 1, 1, S), torch.finfo(torch.float32).min)
    torch.manual_seed(1)
    for t in range(steps):
        x = torch.randn(B, 1, H)
        pos_ids = torch.full((B, 1), t)
        mask[:, :, :, t] = 0.0
        if t == 2:
            mask[1, :, :, 1] = torch.finfo(torch.float32).min   # row 1: position 1 is padding
        cos, sin = rot(x, pos_ids)
        with torch.no_grad():
            y = layer(x, attention_mask=mask, position_ids=pos_ids, past_key_values=cache, use_cache=True,
                      position_embeddings=(cos, sin))
        y = (y[0] if isinstance(y, tuple) else y)[:, 0].numpy()
        got, _ = A.decoder_layer_step(x[:, 0].numpy(), w, t, keys, values, cos[:, 0].numpy(), sin[:, 0].numpy(),
                                      A.additive_mask(mask.numpy(), S), bf16=False)
        assert O.rel_err(got, y) < 2e-5, t
        np.testing.assert_allclose(keys, cache.layers[0].keys.numpy(), rtol=1e-4, atol=1e-5)
        np.testing.assert_allclose(values, cache.layers[0].values.numpy(), rtol=1e-5, atol=1e-6)


def test_attention_matches_transformers_without_qk_norm_and_mha():
    """MHA (G = 1) and no q/k norm: the oracle's attention core alone against
    transformers' eager attention with its rotary embedding."""
    from transformers.models.qwen3.modeling_qwen3 import apply_rotary_pos_emb, eager_attention_forward

    B, HQ, D, S, pos = 2, 4, 64, 10, 6
    rng = _rng(20)
    qkv = rng.standard_normal((B, 3 * HQ * D)).astype(np.float32)
    keys, values = rng.standard_normal((2, B, HQ, S, D)).astype(np.float32)
    theta = rng.uniform(-3, 3, (B, D // 2)).astype(np.float32)
    cos = np.concatenate([np.cos(theta)] * 2, -1)
    sin = np.concatenate([np.sin(theta)] * 2, -1)
    mask = np.where(rng.random((B, S)) < 0.3, np.float32(-1e9), np.float32(0.0))
    mask[:, pos] = 0
    q = A.qkv_rope_cache(qkv, HQ, HQ, D, cos, sin, pos, keys, values, cache_bf16=False)
    got = A.attn_decode(q, keys, values, mask.astype(np.float64), pos)

    qt = torch.from_numpy(qkv[:, : HQ * D].reshape(B, HQ, 1, D))
    kt = torch.from_numpy(qkv[:, HQ * D: 2 * HQ * D].reshape(B, HQ, 1, D))
    qr, kr = apply_rotary_pos_emb(qt, kt, torch.from_numpy(cos)[:, None], torch.from_numpy(sin)[:, None])
    kc = torch.from_numpy(keys.copy())
    np.testing.assert_allclose(kc[:, :, pos], kr[:, :, 0].numpy(), rtol=1e-5, atol=1e-6)

    class _M:
        num_key_value_groups = 1
        training = False

    ref, _ = eager_attention_forward(_M(), qr, kc[:, :, : pos + 1], torch.from_numpy(values[:, :, : pos + 1]),
                                     torch.from_numpy(mask[:, None, None, : pos + 1]), scaling=D ** -0.5)
    assert O.rel_err(got, ref.reshape(B, HQ * D).numpy()) < 1e-5
