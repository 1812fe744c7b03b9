"""Decode attention through the C ABI against the oracle, on the GPU.

Bars: the new k cache entry within one bf16 step of the oracle (the kernel
rounds an fp32 value, the oracle a float64 one), v bit-exact (a copy), q
(fp32) to 1e-5; the attention output, stored as bf16, to 4e-3 of the
largest value (two bf16 roundings) and the reference's 1e-2."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import bz_attn_oracle as A
from oracle import bz_oracle as O
from tests._util import f32

from breeze_amd import attention as T

pytestmark = pytest.mark.gpu

TOL = 1e-2
TIGHT = 4e-3
DEV = "cuda"


def _bf16(a):
    return torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16).to(DEV)


def _case(B, HQ, HKV, D, S, seed, cache_dtype=torch.bfloat16, fill=None):
    """Random qkv (bf16) and a cache already holding `fill` random positions."""
    rng = np.random.default_rng(seed)
    qkv = O.round_bf16(rng.standard_normal((B, (HQ + 2 * HKV) * D)).astype(np.float32) * 2)
    keys = np.zeros((B, HKV, S, D), np.float32)
    values = np.zeros((B, HKV, S, D), np.float32)
    n = S if fill is None else fill
    keys[:, :, :n] = rng.standard_normal((B, HKV, n, D))
    values[:, :, :n] = rng.standard_normal((B, HKV, n, D))
    if cache_dtype == torch.bfloat16:
        keys, values = O.round_bf16(keys), O.round_bf16(values)
    return qkv, keys, values


def _rope_tables(B, D, seed, rows=None):
    rng = np.random.default_rng(seed)
    th = rng.uniform(-4, 4, (rows or B, D // 2)).astype(np.float32)
    return np.concatenate([np.cos(th)] * 2, -1), np.concatenate([np.sin(th)] * 2, -1)


@pytest.mark.parametrize("qk_norm", [True, False])
@pytest.mark.parametrize("cs_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("cache_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("bcast", [False, True])
def test_qkv_rope_cache(qk_norm, cs_dtype, cache_dtype, bcast):
    B, HQ, HKV, D, S, pos = 2, 16, 4, 256, 40, 17
    qkv, keys, values = _case(B, HQ, HKV, D, S, 1, cache_dtype)
    cos, sin = _rope_tables(B, D, 2, rows=1 if bcast else None)
    cos_t = torch.from_numpy(cos).to(cs_dtype).to(DEV)
    sin_t = torch.from_numpy(sin).to(cs_dtype).to(DEV)
    cos, sin = f32(cos_t), f32(sin_t)
    rng = np.random.default_rng(3)
    qn = O.round_bf16(1 + 0.1 * rng.standard_normal(D).astype(np.float32)) if qk_norm else None
    kn = O.round_bf16(1 + 0.1 * rng.standard_normal(D).astype(np.float32)) if qk_norm else None
    kc = torch.from_numpy(keys).to(cache_dtype).to(DEV)
    vc = torch.from_numpy(values).to(cache_dtype).to(DEV)
    counter = torch.zeros((), dtype=torch.int64, device=DEV)
    q = T.qkv_rope_cache(_bf16(qkv), cos_t.unsqueeze(1), sin_t.unsqueeze(1), torch.tensor([pos], device=DEV), kc, vc,
                         HQ, None if qn is None else _bf16(qn), None if kn is None else _bf16(kn), 1e-6,
                         seq_len=counter)
    q_ref = A.qkv_rope_cache(qkv, HQ, HKV, D, cos, sin, pos, keys, values, qn, kn, 1e-6,
                             cache_bf16=cache_dtype == torch.bfloat16)
    assert O.rel_err(f32(q), q_ref) < 1e-5
    got_k, got_v = f32(kc), f32(vc)
    others = [s for s in range(S) if s != pos]
    np.testing.assert_array_equal(got_k[:, :, others], keys[:, :, others])
    np.testing.assert_array_equal(got_v, values)
    step = 2.0 ** -7 if cache_dtype == torch.bfloat16 else 1e-6
    np.testing.assert_allclose(got_k[:, :, pos], keys[:, :, pos], rtol=step, atol=1e-6)
    assert int(counter) == pos + 1


def test_rope_position_outside_cache_writes_nothing():
    B, HQ, HKV, D, S = 1, 4, 2, 64, 8
    qkv, keys, values = _case(B, HQ, HKV, D, S, 4)
    cos, sin = _rope_tables(B, D, 5)
    kc, vc = _bf16(keys), _bf16(values)
    for pos in (S, S + 5, -1):
        T.qkv_rope_cache(_bf16(qkv), _bf16(cos), _bf16(sin), torch.tensor([pos], device=DEV), kc, vc, HQ)
    np.testing.assert_array_equal(f32(kc), keys)
    np.testing.assert_array_equal(f32(vc), values)


SHAPES = [  # (HQ, HKV, D)
    (16, 4, 256), (8, 8, 64), (4, 2, 128), (32, 2, 128), (16, 1, 64), (4, 1, 512), (8, 4, 512), (16, 2, 256),
]


def _attn_check(HQ, HKV, D, S, pos, split, cache_dtype=torch.bfloat16, mask_kind="add_bf16", B=2, seed=0):
    qkv, keys, values = _case(B, HQ, HKV, D, S, seed, cache_dtype)
    rng = np.random.default_rng(seed + 1)
    q = (rng.standard_normal((B, HQ, D)) * 3).astype(np.float32)
    allow = rng.random((B, S)) > 0.15
    allow[:, 0] = True
    if mask_kind == "bool":
        mask_t = torch.from_numpy(allow.reshape(B, 1, 1, S)).to(DEV)
        madd = A.additive_mask(allow, S)
    elif mask_kind == "bcast":
        m = np.where(allow[:1], 0.0, np.float32(-1e9)).astype(np.float32)
        mask_t = torch.from_numpy(m.reshape(1, 1, 1, S)).to(DEV)
        madd = np.broadcast_to(m.astype(np.float64), (B, S))
    else:
        dt = torch.bfloat16 if mask_kind == "add_bf16" else torch.float32
        m = np.where(allow, 0.0, float(torch.finfo(dt).min))
        mask_t = torch.from_numpy(m.reshape(B, 1, 1, S)).to(dt).to(DEV)
        madd = m
    kc = torch.from_numpy(keys).to(cache_dtype).to(DEV)
    vc = torch.from_numpy(values).to(cache_dtype).to(DEV)
    out = T.attn_decode(torch.from_numpy(q).to(DEV), kc, vc, mask_t, torch.tensor([pos], device=DEV), split=split)
    ref = A.attn_decode(q, keys, values, madd, pos)
    got = f32(out)
    assert O.rel_err(got, ref) <= TIGHT, (O.rel_err(got, ref), HQ, HKV, D, S, pos, split)
    assert np.isfinite(got).all()
    return got


@pytest.mark.parametrize("HQ,HKV,D", SHAPES)
@pytest.mark.parametrize("pos,split", [(0, 1), (15, 1), (16, 1), (63, 1), (63, 3), (200, 8), (511, 4),
                                       (511, None)])
def test_attn_decode_shapes(HQ, HKV, D, pos, split):
    _attn_check(HQ, HKV, D, 512, pos, split)


@pytest.mark.parametrize("HQ,HKV,D", [(16, 4, 256), (8, 2, 128), (4, 2, 128), (8, 8, 64), (16, 16, 64)])
@pytest.mark.parametrize("S,pos", [(1, 0), (16, 0), (16, 15), (17, 16), (17, 9), (32, 31), (32, 16), (33, 32)])
@pytest.mark.parametrize("split", [1, 3])
def test_attn_decode_short_cache(HQ, HKV, D, S, pos, split):
    """Caches of at most 33 positions (the depth decoder's hold 17): one or
    two 16-position blocks, the rest of the workgroup's waves idle until the
    merge."""
    _attn_check(HQ, HKV, D, S, pos, split, seed=S + pos)


@pytest.mark.parametrize("cache_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("mask_kind", ["add_bf16", "add_f32", "bool", "bcast"])
def test_attn_decode_dtypes_and_masks(cache_dtype, mask_kind):
    _attn_check(16, 4, 256, 300, 250, 4, cache_dtype, mask_kind)
    _attn_check(8, 2, 128, 48, 47, 1, cache_dtype, mask_kind, B=3)


@pytest.mark.parametrize("split", [1, 2, 7, 16, 64])
def test_attn_split_counts_agree(split):
    """Every split count (including splits left empty: 64 splits over 40
    positions) gives the unsplit result."""
    a = _attn_check(16, 4, 256, 128, 39, split, seed=7)
    b = _attn_check(16, 4, 256, 128, 39, 1, seed=7)
    assert O.rel_err(a, b) <= TIGHT


@pytest.mark.parametrize("pos,split", [(159, 8), (160, 8), (191, 8), (193, 64), (250, 64)])
def test_attn_unsplit_threshold_and_empty_splits(pos, split):
    """Around the on-device unsplit threshold (160 attended positions: pos 159
    runs unsplit, pos 160 splits), and splits left empty above it (64 splits
    over 194 / 251 positions: per = 4, the last splits hold nothing) with the
    cross-workgroup combine: all equal the unsplit result."""
    a = _attn_check(16, 4, 256, 512, pos, split, seed=13)
    b = _attn_check(16, 4, 256, 512, pos, 1, seed=13)
    assert O.rel_err(a, b) <= TIGHT


def test_attn_large_cache_full_length():
    _attn_check(16, 4, 256, 2048, 2047, None, B=2, seed=11)


def test_attn_one_position_returns_value_row():
    B, HQ, HKV, D, S = 2, 16, 4, 256, 64
    _, keys, values = _case(B, HQ, HKV, D, S, 12)
    q = torch.randn(B, HQ, D, device=DEV)
    mask = torch.zeros(B, 1, 1, S, device=DEV)
    out = T.attn_decode(q, _bf16(keys), _bf16(values), mask, torch.tensor([0], device=DEV)).view(B, HQ, D)
    for h in range(HQ):
        np.testing.assert_array_equal(f32(out[:, h]), values[:, h // 4, 0])


def test_attn_position_outside_cache():
    B, HQ, HKV, D, S = 1, 8, 2, 128, 32
    qkv, keys, values = _case(B, HQ, HKV, D, S, 13)
    q = torch.randn(B, HQ, D, device=DEV)
    mask = torch.zeros(B, 1, 1, S, device=DEV)
    kc, vc = _bf16(keys), _bf16(values)
    out = T.attn_decode(q, kc, vc, mask, torch.tensor([-1], device=DEV))
    assert not f32(out).any()
    big = T.attn_decode(q, kc, vc, mask, torch.tensor([S + 100], device=DEV), split=1)
    full = T.attn_decode(q, kc, vc, mask, torch.tensor([S - 1], device=DEV), split=1)
    np.testing.assert_array_equal(f32(big), f32(full))


@pytest.mark.parametrize("HQ,HKV,D", [(16, 4, 256), (8, 2, 128), (16, 1, 64), (4, 1, 512)])
@pytest.mark.parametrize("pos,S,split", [(0, 64, 1), (37, 64, 1), (37, 64, 4), (511, 512, None), (300, 512, 16),
                                         (0, 17, 1), (16, 17, 1), (31, 32, 2)])
@pytest.mark.parametrize("qk_norm", [True, False])
def test_attention_step_fused_matches_oracle_and_unfused(HQ, HKV, D, pos, S, split, qk_norm):
    """One launch of bz_attn_step against the oracle's rope + cache write +
    attention, and against qkv_rope_cache + attn_decode (the same arithmetic
    in two launches: bit-identical for D <= 256, where both sum the head
    norm in the same order)."""
    B = 2
    qkv, keys, values = _case(B, HQ, HKV, D, S, 30 + pos, fill=pos)
    cos, sin = (O.round_bf16(t) for t in _rope_tables(B, D, 31))   # the tables the GPU gets, as bf16
    rng = np.random.default_rng(32)
    qn = O.round_bf16(1 + 0.1 * rng.standard_normal(D).astype(np.float32)) if qk_norm else None
    kn = O.round_bf16(1 + 0.1 * rng.standard_normal(D).astype(np.float32)) if qk_norm else None
    allow = rng.random((B, S)) > 0.1
    allow[:, pos] = True
    mask = np.where(allow, 0.0, float(torch.finfo(torch.bfloat16).min))
    mask_t = torch.from_numpy(mask.reshape(B, 1, 1, S)).to(torch.bfloat16).to(DEV)
    args = (_bf16(cos), _bf16(sin), torch.tensor([pos], device=DEV))
    nw = (None if qn is None else _bf16(qn), None if kn is None else _bf16(kn))
    kc, vc = _bf16(keys), _bf16(values)
    kc2, vc2 = kc.clone(), vc.clone()
    counter = torch.zeros((), dtype=torch.int64, device=DEV)
    out = T.attention_step(_bf16(qkv), *args, kc, vc, mask_t, *nw, 1e-6, split=split, seq_len=counter)
    q = T.qkv_rope_cache(_bf16(qkv), *args, kc2, vc2, HQ, *nw, 1e-6)
    out2 = T.attn_decode(q, kc2, vc2, mask_t, args[2], split=split)
    assert int(counter) == pos + 1
    np.testing.assert_array_equal(f32(kc), f32(kc2))
    np.testing.assert_array_equal(f32(vc), f32(vc2))
    if D <= 256:
        np.testing.assert_array_equal(f32(out), f32(out2))
    q_ref = A.qkv_rope_cache(qkv, HQ, HKV, D, cos, sin, pos, keys, values, qn, kn, 1e-6)
    ref = A.attn_decode(q_ref, keys, values, mask, pos)
    assert O.rel_err(f32(out), ref) <= TIGHT
    step = 2.0 ** -7
    np.testing.assert_allclose(f32(kc)[:, :, pos], keys[:, :, pos], rtol=step, atol=1e-6)


def test_attention_step_workspace_reuse_across_shapes_and_calls():
    """Many calls in a row with split > 1 (the arrival counters must return
    to zero after every call) at changing positions, two batch sizes."""
    HQ, HKV, D, S = 16, 4, 256, 256
    for B in (1, 2):
        qkv, keys, values = _case(B, HQ, HKV, D, S, 40 + B)
        cos, sin = (O.round_bf16(t) for t in _rope_tables(B, D, 41))
        mask_t = torch.zeros(B, 1, 1, S, device=DEV)
        kc, vc = _bf16(keys), _bf16(values)
        for pos in (255, 3, 100, 0, 200, 255, 17):
            kref, vref = f32(kc), f32(vc)
            out = T.attention_step(_bf16(qkv), _bf16(cos), _bf16(sin), torch.tensor([pos], device=DEV), kc, vc,
                                   mask_t, split=8)
            q_ref = A.qkv_rope_cache(qkv, HQ, HKV, D, cos, sin, pos, kref, vref)
            assert O.rel_err(f32(out), A.attn_decode(q_ref, kref, vref, np.zeros((B, S)), pos)) <= TIGHT, (B, pos)


def test_attention_step_graph_replays_track_device_position():
    """attention_step captured once in a HIP graph, replayed with the device
    position and mask updated between replays: every replay equals an eager
    call on a cache copy."""
    B, HQ, HKV, D, S = 2, 16, 4, 256, 192
    qkv, keys, values = _case(B, HQ, HKV, D, S, 14, fill=0)
    cos, sin = _rope_tables(B, D, 15)
    qkv_t, cos_t, sin_t = _bf16(qkv), _bf16(cos), _bf16(sin)
    kc, vc = _bf16(keys), _bf16(values)
    kc2, vc2 = kc.clone(), vc.clone()
    pos = torch.zeros(1, dtype=torch.int64, device=DEV)
    mask = torch.full((B, 1, 1, S), float(torch.finfo(torch.bfloat16).min), dtype=torch.bfloat16, device=DEV)
    out = torch.empty(B, HQ * D, dtype=torch.bfloat16, device=DEV)
    qbuf = torch.empty(B, HQ, D, device=DEV)
    step = lambda k, v, o, qb: T.attention_step(qkv_t, cos_t, sin_t, pos, k, v, mask, out=o, q_buf=qb)  # noqa: E731
    step(kc, vc, out, qbuf)
    torch.cuda.synchronize()
    kc.zero_()
    vc.zero_()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st):
        with torch.cuda.graph(g, stream=st):
            step(kc, vc, out, qbuf)
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    for t in range(0, 190, 11):
        pos.fill_(t)
        mask[:, :, :, : t + 1] = 0
        qkv_t.copy_(_bf16(np.random.default_rng(t).standard_normal(qkv.shape) * 2))
        g.replay()
        ref = step(kc2, vc2, None, None)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(f32(out), f32(ref))
        np.testing.assert_array_equal(f32(kc), f32(kc2))
