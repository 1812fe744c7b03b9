"""CPU oracle for the decode attention step and the fused decoder layer
(test infrastructure only).

Like ``bz_oracle`` this is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import it.

Restated from the reference:

* ``rms_head``          models/fused/kernels.py:356-359  per-head RMSNorm in
                        fp32, v * (1/sqrt(mean(v^2)+eps)) * w
* ``rotate_half`` / ``rope``  models/fused/kernels.py:362-373 and
                        models/breeze.py:197-228 (v*cos + [-v2, v1]*sin)
* ``qkv_rope_cache``    models/fused/kernels.py:376-401  q heads -> fp32 q,
                        kv heads -> k (normed, rotated) and v into the static
                        cache at position pos, rounded to the cache dtype
* ``additive_mask``     models/fused/kernels.py:492-502  bool -> 0 / -1e30
* ``attn_decode``       models/fused/kernels.py:404-453 (+ combine :456-475)
                        softmax(q k^T * D^-0.5 + mask) v over positions
                        [0, pos], query head h reading kv head h // (HQ/HKV)
* ``attn_decode_split`` the split-S partials (acc, m, l) and their combine,
                        models/fused/kernels.py:437-475
* ``decoder_layer_step`` models/fused/layer.py:83-98  one decode step of a
                        decoder layer: rmsnorm -> qkv -> attention -> o_proj
                        + residual -> rmsnorm -> silu(gate) * up -> down +
                        residual, with the weights given as dense fp32
                        matrices (the dequantized w_eff for int4 / fp8)

Arithmetic is float64 except where the reference rounds (k and v stored in
the cache dtype, bf16 activations between GEMVs), so the oracle sits at
least as close to exact as the reference's fp32 kernels.

Pinning (tests/test_attn_oracle.py):
  qkv_rope_cache, attn_decode, decoder_layer_step
      - transformers' own Qwen3 decoder layer (the reference's unfused path,
        eager attention, StaticCache) on the CPU in float32, several decode
        steps with GQA, q/k norm and a padded additive mask;
  rope    - cos = 1, sin = 0 is the identity; a rotation keeps every (d,
            d + D/2) pair's norm; rotate_half applied twice negates;
  attn    - one attended position returns its value row; equal keys give
            the mean of the attended values; a -1e30 mask entry equals
            dropping the position; additive constant on all scores changes
            nothing; brute-force float64 loop on a tiny case;
  split   - the split partials combine to the unsplit result for every split
            count, including empty splits.
No function here is "parity unpinned".
"""

from __future__ import annotations

import numpy as np

from .bz_oracle import (
    EPI_RES,
    EPI_SILU,
    bf16_bits_to_f32,
    f32_to_bf16_bits,
    gemv_ref,
    rmsnorm_f32,
    round_bf16,
)

NEG_BIG = -1e30


def rms_head(v, w, eps: float):
    """models/fused/kernels.py:356-359 (v [..., D], w [D])."""
    v = np.asarray(v, np.float64)
    var = np.mean(v * v, axis=-1, keepdims=True)
    return v / np.sqrt(var + eps) * np.asarray(w, np.float64)


def rotate_half(v):
    """[-v2, v1] over the last axis (models/breeze.py:197-201)."""
    v = np.asarray(v)
    h = v.shape[-1] // 2
    return np.concatenate([-v[..., h:], v[..., :h]], axis=-1)


def rope(v, cos, sin):
    """v * cos + rotate_half(v) * sin (models/fused/kernels.py:362-373)."""
    return np.asarray(v, np.float64) * cos + rotate_half(np.asarray(v, np.float64)) * sin


def qkv_rope_cache(qkv, HQ: int, HKV: int, D: int, cos, sin, pos: int, keys, values, qn=None, kn=None,
                   eps: float = 1e-6, cache_bf16: bool = True):
    """qkv float [B, (HQ + 2 HKV) D] (bf16 values) -> q float64 [B, HQ, D];
    writes k and v at cache position ``pos`` of keys/values [B, HKV, S, D]
    (float arrays, values rounded to bf16 when ``cache_bf16``).  cos/sin are
    [B or 1, D].  models/fused/kernels.py:376-401."""
    qkv = np.asarray(qkv, np.float64)
    B = qkv.shape[0]
    cos = np.broadcast_to(np.asarray(cos, np.float64).reshape(-1, D), (B, D))[:, None, :]
    sin = np.broadcast_to(np.asarray(sin, np.float64).reshape(-1, D), (B, D))[:, None, :]
    q = qkv[:, : HQ * D].reshape(B, HQ, D)
    k = qkv[:, HQ * D: (HQ + HKV) * D].reshape(B, HKV, D)
    v = qkv[:, (HQ + HKV) * D:].reshape(B, HKV, D)
    if qn is not None:
        q = rms_head(q, qn, eps)
        k = rms_head(k, kn, eps)
    q = rope(q, cos, sin)
    k = rope(k, cos, sin)
    S = keys.shape[2]
    if 0 <= pos < S:
        keys[:, :, pos] = round_bf16(k) if cache_bf16 else k.astype(np.float32)
        values[:, :, pos] = v
    return q


def additive_mask(mask, S: int):
    """(B, ..., >= S) bool or additive -> (B, S) float64
    (models/fused/kernels.py:492-502)."""
    m = np.asarray(mask)
    m = m.reshape(m.shape[0], -1)[:, :S]
    if m.dtype == np.bool_:
        return np.where(m, 0.0, NEG_BIG)
    return m.astype(np.float64)


def attn_decode(q, keys, values, mask_add, pos: int, scale=None):
    """q [B, HQ, D] -> out float64 [B, HQ * D]; softmax over positions
    [0, pos] of q k^T * scale + mask (models/fused/kernels.py:404-453)."""
    q = np.asarray(q, np.float64)
    B, HQ, D = q.shape
    HKV, S = keys.shape[1], keys.shape[2]
    G = HQ // HKV
    scale = D ** -0.5 if scale is None else scale
    n = min(pos + 1, S)
    out = np.zeros((B, HQ, D))
    for b in range(B):
        for h in range(HQ):
            kk = np.asarray(keys[b, h // G, :n], np.float64)
            vv = np.asarray(values[b, h // G, :n], np.float64)
            s = kk @ (q[b, h] * scale) + mask_add[b, :n]
            p = np.exp(s - s.max())
            out[b, h] = (p @ vv) / p.sum()
    return out.reshape(B, HQ * D)


def attn_decode_split(q, keys, values, mask_add, pos: int, split: int, scale=None):
    """The same through split-S partials (acc, m, l) with running max
    initialised to -1e30, then the combine (models/fused/kernels.py:425-475)."""
    q = np.asarray(q, np.float64)
    B, HQ, D = q.shape
    HKV, S = keys.shape[1], keys.shape[2]
    G = HQ // HKV
    scale = D ** -0.5 if scale is None else scale
    kv_len = min(pos + 1, S)
    per = -(-kv_len // split)
    out = np.zeros((B, HQ, D))
    for b in range(B):
        for h in range(HQ):
            parts = []
            for sp in range(split):
                lo, hi = sp * per, min(sp * per + per, kv_len)
                m, l, acc = NEG_BIG, 0.0, np.zeros(D)
                if hi > lo:
                    kk = np.asarray(keys[b, h // G, lo:hi], np.float64)
                    vv = np.asarray(values[b, h // G, lo:hi], np.float64)
                    s = kk @ (q[b, h] * scale) + mask_add[b, lo:hi]
                    m = max(m, s.max())
                    p = np.exp(s - m)
                    l, acc = p.sum(), p @ vv
                parts.append((m, l, acc))
            mt = max(p[0] for p in parts)
            w = [np.exp(p[0] - mt) for p in parts]
            out[b, h] = sum(wi * p[2] for wi, p in zip(w, parts)) / sum(wi * p[1] for wi, p in zip(w, parts))
    return out.reshape(B, HQ * D)


def decoder_layer_step(x, w, pos: int, keys, values, cos, sin, mask_add, eps: float = 1e-6, bf16: bool = True):
    """One decode step of a decoder layer (models/fused/layer.py:83-98).

    x bf16-valued float [B, H]; w: dict with ``ln1``, ``ln2`` [H], ``qn``,
    ``kn`` [D] or None, dense fp32 ``wqkv`` [(HQ + 2 HKV) D, H], ``wo``
    [H, HQ D], ``wgu`` [2 I, H] ([gate; up]), ``wd`` [H, I], and ints ``HQ``,
    ``HKV``, ``D``.  With ``bf16`` the activations between GEMVs and the
    cache are rounded to bf16 as on the fused path; without, everything stays
    float (the form that matches a float32 model).  Returns (out float32
    [B, H], q)."""
    HQ, HKV, D = w["HQ"], w["HKV"], w["D"]
    r = round_bf16 if bf16 else (lambda v: np.asarray(v, np.float32))
    x = np.asarray(x, np.float32)
    qkv = r(gemv_ref(rmsnorm_f32(x, w["ln1"], eps), w["wqkv"]))
    q = qkv_rope_cache(qkv, HQ, HKV, D, cos, sin, pos, keys, values, w.get("qn"), w.get("kn"), eps, cache_bf16=bf16)
    attn = r(attn_decode(q, keys, values, mask_add, pos).astype(np.float32))
    h = r(gemv_ref(attn, w["wo"], EPI_RES, x))
    act = r(gemv_ref(rmsnorm_f32(h, w["ln2"], eps), w["wgu"], EPI_SILU))
    out = gemv_ref(act, w["wd"], EPI_RES, h)
    return out.astype(np.float32), q


__all__ = [
    "NEG_BIG",
    "rms_head",
    "rotate_half",
    "rope",
    "qkv_rope_cache",
    "additive_mask",
    "attn_decode",
    "attn_decode_split",
    "decoder_layer_step",
    "bf16_bits_to_f32",
    "f32_to_bf16_bits",
]
