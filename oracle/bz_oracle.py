"""CPU oracle for the decode-time linear layers (test infrastructure only).

This module is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The GPU path lives in ``breeze-tts-2_amd/`` and must never route
through here.

It restates, in plain numpy with explicit IEEE float32 steps, the algorithm of
the reference's decode linears:

* ``quantize_int4_asym``   models/int4_linear.py:47-64 (min/max, (q-8)*s+z form)
* ``quantize_int4_sym``    symmetric group-128 variant (absmax/7, z = 0)
* ``pack_nibbles_*``       models/int4_linear.py:57-58 (odd-k low nibble) and
                           models/fused/kernels.py:149 (even-k low nibble)
* ``pack_int4_fused``      models/fused/kernels.py:141-150 (q*s+min form)
* ``quantize_fp8_linear``  models/fp8_linear.py:56-66 (amax floor 1e-12)
* ``pack_fp8``             models/fused/kernels.py:153-158 (amax floor 1e-8)
* ``e4m3fn_decode`` / ``e4m3fn_encode``  OCP FP8 E4M3 (the torch float8_e4m3fn
                           format the reference casts to)
* ``rmsnorm_*``            models/fused/kernels.py:65-81 (fp32 x_hat),
                           models/breeze.py:115-120 (model RMSNorm rounding),
                           bench_gemv.py:31 (bf16-rounded x_hat)
* ``gemv_ref``             models/fused/kernels.py:74-104 + 107-138 and the
                           dequantize-then-matmul definition bench_gemv.py:30-53
* ``linear_f32_ref``       fp32 lm_head, models/cudagraph/backbone_graph.py:69-70,273
* ``codebooks_head_ref``   BreezeCodebooksHead.forward, models/breeze.py:597-612
* ``rel_err``              bench_gemv.py:53  max|out-ref| / max|ref|
* ``tile_int4`` / ``tile_fp8`` and their inverses: this build's row-block
                           tiled weight layout (no reference counterpart: it
                           replaces tinygemm's opaque repack,
                           models/int4_linear.py:59), restated byte by byte
                           from its written definition in include/bz_gemv.h

bfloat16 is handled as raw uint16 bit patterns (numpy has no bf16 dtype).
Every rounding to bf16 is round-to-nearest-even, as torch's ``.to(bfloat16)``.

Pinning (what checks each function; see tests/test_oracle.py):
  quantizers   - closed forms on constant groups (scale floor), on-grid weights
                 recovered exactly, RNE ties, brute-force per-element loop
  nibble packs - single-nonzero-nibble sweeps, pack/unpack round trips,
                 committed golden vectors
  e4m3fn       - all 256 codes decoded from the bit-field definition and
                 cross-checked against torch's CPU float8_e4m3fn cast
                 (a library, not the reference); encode checked against the
                 same cast on a dense sweep, including ties and subnormals
  rmsnorm      - float64 brute force, scale invariance rms(c*x) = rms(x)
  gemv         - float64 brute-force loops on tiny shapes, linearity in x,
                 one-hot x selects one weight column, zero W gives 0 (+res)
  epilogues    - closed forms of SiLU(g)*u and +residual
  fp32 heads   - torch's CPU float64 linear per codebook (a library routine);
                 codebook selection by one-hot weights naming their codebook
  tiled layout - untile(tile(x)) = x, every byte of a source lands at the
                 offset a scalar loop over the definition computes, the paired
                 order puts gate/up rows 8b+r in tile rows r and 8+r
No function here is "parity unpinned": the reference publishes no golden
vectors for this path (it has no automated test of it), so the pins above are
the mathematics plus committed fixtures produced by this file.
"""

from __future__ import annotations

import numpy as np

GROUP = 128
FP8_MAX = 448.0

# ----------------------------------------------------------------------------
# bfloat16 as uint16 bit patterns
# ----------------------------------------------------------------------------


def f32_to_bf16_bits(a) -> np.ndarray:
    """float32 -> bf16 bit pattern, round to nearest even (NaN kept quiet)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32)
    nan = np.isnan(a)
    rounded = np.where(nan, ((u >> 16) | 0x40).astype(np.uint32), rounded)
    return rounded.astype(np.uint16)


def bf16_bits_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def round_bf16(a) -> np.ndarray:
    """Round float32 values to the nearest bf16 value, returned as float32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(a))


# ----------------------------------------------------------------------------
# OCP FP8 E4M3 ("fn": no infinities, 0x7F/0xFF are NaN, max 448)
# ----------------------------------------------------------------------------


def e4m3fn_decode_table() -> np.ndarray:
    """Value of each of the 256 codes, from the bit-field definition:
    sign | 4-bit exponent (bias 7) | 3-bit mantissa; exponent 0 is subnormal
    (m/8 * 2^-6); S.1111.111 is NaN; there is no infinity."""
    out = np.empty(256, dtype=np.float32)
    for code in range(256):
        s = -1.0 if code & 0x80 else 1.0
        e = (code >> 3) & 0xF
        m = code & 0x7
        if e == 0xF and m == 0x7:
            out[code] = np.nan
        elif e == 0:
            out[code] = s * (m / 8.0) * 2.0 ** -6
        else:
            out[code] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return out


_E4M3_TABLE = e4m3fn_decode_table()
# Non-negative finite codes 0x00..0x7E in increasing value order.
_E4M3_POS = _E4M3_TABLE[:0x7F].astype(np.float64)


def e4m3fn_decode(codes) -> np.ndarray:
    return _E4M3_TABLE[np.asarray(codes, dtype=np.uint8)]


def e4m3fn_encode(a) -> np.ndarray:
    """float32 -> e4m3fn code, round to nearest, ties to the even code.

    Restated as a nearest-neighbour search over the 127 non-negative finite
    values (not the bit trick the device code uses).  Inputs must already be
    clamped to [-448, 448] as the reference does before its cast
    (models/fp8_linear.py:60, models/fused/kernels.py:157); NaN maps to 0x7F.
    """
    a = np.asarray(a, dtype=np.float32)
    mag = np.abs(a).astype(np.float64)
    if np.any(mag[~np.isnan(mag)] > FP8_MAX):
        raise ValueError("e4m3fn_encode expects inputs clamped to +-448")
    hi = np.searchsorted(_E4M3_POS, mag, side="left")
    hi = np.clip(hi, 0, 0x7E)
    lo = np.clip(hi - 1, 0, 0x7E)
    d_hi = np.abs(_E4M3_POS[hi] - mag)
    d_lo = np.abs(mag - _E4M3_POS[lo])
    pick = np.where(d_lo < d_hi, lo, hi)
    tie = (d_lo == d_hi) & (lo != hi)
    pick = np.where(tie, np.where(lo % 2 == 0, lo, hi), pick)
    code = pick.astype(np.uint8)
    neg = np.signbit(a)
    code = np.where(neg, code | 0x80, code).astype(np.uint8)
    code = np.where(np.isnan(a), np.uint8(0x7F), code).astype(np.uint8)
    return code


# ----------------------------------------------------------------------------
# int4 quantizers
# ----------------------------------------------------------------------------


def quantize_int4_asym(w, group: int = GROUP):
    """models/int4_linear.py:47-63 (also bench_int4_shapes.py:46-68).

    Per (row n, group of `group` consecutive k):
        lo = min, hi = max
        s  = max((hi - lo) / 15, 1e-8)          (float32)
        q  = clamp(rne((w - lo) / s), 0, 15)    (float32 divide, RNE)
        z  = lo + 8 s                           (the (q-8)*s+z zero point)
    Returns q uint8 [N,K], s float32 [N,G], lo float32 [N,G], z float32 [N,G].
    The stored scales_zeros rounds s and z to bf16 (see ``scales_zeros``).
    """
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    if k % group:
        raise ValueError(f"in_features {k} not divisible by group {group}")
    g = w.reshape(n, k // group, group)
    lo = g.min(axis=-1, keepdims=True)
    hi = g.max(axis=-1, keepdims=True)
    s = np.maximum((hi - lo) / np.float32(15.0), np.float32(1e-8)).astype(np.float32)
    q = np.clip(np.rint((g - lo) / s), 0, 15).astype(np.uint8).reshape(n, k)
    z = (lo + np.float32(8.0) * s).astype(np.float32)
    return q, s[..., 0], lo[..., 0], z[..., 0]


def quantize_int4_sym(w, group: int = GROUP):
    """Symmetric group quantizer (the special case z = 0 of the (q-8)*s+z
    form used by models/int4_linear.py:61-63):
        s = max(absmax / 7, 1e-8);  q = clamp(rne(w / s) + 8, 0, 15);  z = 0
    Returns q uint8 [N,K], s float32 [N,G], z float32 [N,G] (zeros)."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    if k % group:
        raise ValueError(f"in_features {k} not divisible by group {group}")
    g = w.reshape(n, k // group, group)
    amax = np.abs(g).max(axis=-1, keepdims=True)
    s = np.maximum(amax / np.float32(7.0), np.float32(1e-8)).astype(np.float32)
    q = np.clip(np.rint(g / s) + 8, 0, 15).astype(np.uint8).reshape(n, k)
    return q, s[..., 0], np.zeros_like(s[..., 0])


def scales_zeros(s, z) -> np.ndarray:
    """[N,G] scale and zero -> [G,N,2] bf16 bits, as
    torch.stack([s.t(), z.t()], -1).to(bfloat16) (models/int4_linear.py:61-63)."""
    s = np.asarray(s, dtype=np.float32).T
    z = np.asarray(z, dtype=np.float32).T
    return f32_to_bf16_bits(np.stack([s, z], axis=-1))


def pack_int4_fused(w, group: int = GROUP):
    """models/fused/kernels.py:141-150: same min/max quantizer, scale and min
    stored separately as [N, K/g] bf16; dequant w = q*s + min.
    Returns (packed uint8 [N,K/2] even-k-low, scale bf16 bits, min bf16 bits)."""
    q, s, lo, _ = quantize_int4_asym(w, group)
    return pack_nibbles_even_low(q), f32_to_bf16_bits(s), f32_to_bf16_bits(lo)


# ----------------------------------------------------------------------------
# nibble packing
# ----------------------------------------------------------------------------


def pack_nibbles_odd_low(q) -> np.ndarray:
    """models/int4_linear.py:57-58: byte j = q[2j+1] | q[2j] << 4."""
    q = np.asarray(q, dtype=np.uint8)
    return (q[:, 1::2] | (q[:, 0::2] << 4)).astype(np.uint8)


def pack_nibbles_even_low(q) -> np.ndarray:
    """models/fused/kernels.py:149: byte j = q[2j] | q[2j+1] << 4.
    This is also the byte layout of the GPU path's ``weight_int4``."""
    q = np.asarray(q, dtype=np.uint8)
    return (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)


def unpack_nibbles_even_low(packed) -> np.ndarray:
    """bench_gemv.py:51: stack([w & 15, w >> 4], -1).reshape(N, K)."""
    p = np.asarray(packed, dtype=np.uint8)
    n = p.shape[0]
    return np.stack([p & 15, p >> 4], axis=-1).reshape(n, -1).astype(np.uint8)


def unpack_nibbles_odd_low(packed) -> np.ndarray:
    p = np.asarray(packed, dtype=np.uint8)
    n = p.shape[0]
    return np.stack([p >> 4, p & 15], axis=-1).reshape(n, -1).astype(np.uint8)


# ----------------------------------------------------------------------------
# dequantization (the W_eff of bench_gemv.py:47-52)
# ----------------------------------------------------------------------------


def dequant_int4_zp(q, sz_bits, group: int = GROUP) -> np.ndarray:
    """w = (q - 8) * s + z with s, z the bf16 values of scales_zeros [G,N,2]
    (the tinygemm semantics documented at models/int4_linear.py:26-28).
    float32 arithmetic: (q-8)*s is exact (|q-8| <= 8, s has 8 significant
    bits), then one rounding for the add."""
    q = np.asarray(q, dtype=np.uint8)
    n, k = q.shape
    sz = bf16_bits_to_f32(sz_bits)  # [G, N, 2]
    s = np.ascontiguousarray(sz[..., 0].T)[:, :, None]  # [N, G, 1], broadcast over the group's k
    z = np.ascontiguousarray(sz[..., 1].T)[:, :, None]
    qg = q.reshape(n, k // group, group).astype(np.float32)
    return ((qg - np.float32(8.0)) * s + z).reshape(n, k).astype(np.float32, copy=False)


def dequant_int4_min(q, s_bits, m_bits, group: int = GROUP) -> np.ndarray:
    """w = q * s + min with [N, K/g] bf16 scale and min
    (models/fused/kernels.py:89-95, bench_gemv.py:51-52)."""
    q = np.asarray(q, dtype=np.uint8)
    s = np.repeat(bf16_bits_to_f32(s_bits), group, axis=1)
    m = np.repeat(bf16_bits_to_f32(m_bits), group, axis=1)
    return (q.astype(np.float32) * s + m).astype(np.float32)


# ----------------------------------------------------------------------------
# fp8 quantizers
# ----------------------------------------------------------------------------


def _fp8_quant(w, floor: float):
    w = np.asarray(w, dtype=np.float32)
    amax = np.maximum(np.abs(w).max(axis=1, keepdims=True), np.float32(floor)).astype(np.float32)
    scale = (amax / np.float32(FP8_MAX)).astype(np.float32)
    v = np.clip(w / scale, -FP8_MAX, FP8_MAX).astype(np.float32)
    return e4m3fn_encode(v), scale[:, 0]


def quantize_fp8_linear(w):
    """models/fp8_linear.py:58-62: amax.clamp(min=1e-12), scale = amax/448,
    clamp(w/scale, +-448) -> e4m3fn.  Returns (codes uint8 [N,K], scale f32 [N])."""
    return _fp8_quant(w, 1e-12)


def pack_fp8(w):
    """models/fused/kernels.py:153-158: same with amax.clamp_min(1e-8)."""
    return _fp8_quant(w, 1e-8)


def dequant_fp8(codes, scale) -> np.ndarray:
    """bench_gemv.py:49: w8.float() * s[:, None]."""
    return (e4m3fn_decode(codes) * np.asarray(scale, dtype=np.float32)[:, None]).astype(np.float32)


# ----------------------------------------------------------------------------
# RMSNorm variants
# ----------------------------------------------------------------------------


def _inv_rms(x, eps):
    x = np.asarray(x, dtype=np.float32)
    ms = (x.astype(np.float64) ** 2).mean(axis=-1, keepdims=True)
    return (1.0 / np.sqrt(ms + eps)).astype(np.float32)


def rmsnorm_f32(x, gamma, eps: float = 1e-6) -> np.ndarray:
    """Fused-kernel semantics (models/fused/kernels.py:65-81): fp32 x_hat =
    x * rsqrt(mean(x^2) + eps) * gamma, no bf16 rounding."""
    x = np.asarray(x, dtype=np.float32)
    g = np.asarray(gamma, dtype=np.float32)
    return (x * _inv_rms(x, eps) * g).astype(np.float32)


def rmsnorm_bf16(x, gamma, eps: float = 1e-6) -> np.ndarray:
    """Standalone-norm rounding: x_hat = bf16(x * inv_rms * gamma)."""
    return round_bf16(rmsnorm_f32(x, gamma, eps))


def rmsnorm_folded(x, gamma, eps: float = 1e-6) -> np.ndarray:
    """Rounding of the fused norm-GEMV: the product is taken against
    u = bf16(x * gamma) and scaled by inv_rms afterwards, which equals a GEMV
    over x_hat = u * inv_rms (fp32, no second rounding)."""
    x = np.asarray(x, dtype=np.float32)
    u = round_bf16(x * np.asarray(gamma, dtype=np.float32))
    return (u * _inv_rms(x, eps)).astype(np.float32)


def rmsnorm_model(x, gamma, eps: float = 1e-6) -> np.ndarray:
    """BreezeRMSNorm (models/breeze.py:115-120): bf16(gamma * bf16(x*inv))."""
    x = np.asarray(x, dtype=np.float32)
    h = round_bf16(x * _inv_rms(x, eps))
    return round_bf16(np.asarray(gamma, dtype=np.float32) * h)


# ----------------------------------------------------------------------------
# GEMV + epilogues
# ----------------------------------------------------------------------------

EPI_NONE, EPI_SILU, EPI_RES = 0, 1, 2


def silu(v):
    v = np.asarray(v, dtype=np.float64)
    return v / (1.0 + np.exp(-v))


def gemv_ref(xn, w_eff, epilogue: int = EPI_NONE, residual=None, row_scale=None) -> np.ndarray:
    """out = epilogue(xn @ W_eff^T) in float64 (bench_gemv.py:30-35).

    row_scale  : fp8 per-output-channel scale applied before the epilogue
                 (models/fused/kernels.py:124-126, 133-134); None when W_eff
                 already includes it.
    EPI_SILU   : silu(acc[:, :N/2]) * acc[:, N/2:] (kernels.py:116-127)
    EPI_RES    : acc + residual (kernels.py:135-136)
    """
    xn = np.asarray(xn, dtype=np.float64)
    w = np.asarray(w_eff, dtype=np.float64)
    acc = xn @ w.T
    if row_scale is not None:
        acc = acc * np.asarray(row_scale, dtype=np.float64)[None, :]
    if epilogue == EPI_SILU:
        h = acc.shape[1] // 2
        return silu(acc[:, :h]) * acc[:, h:]
    if epilogue == EPI_RES:
        return acc + np.asarray(residual, dtype=np.float64)
    return acc


def linear_f32_ref(x, w) -> np.ndarray:
    """The fp32 lm_head: float64 x @ W^T (models/cudagraph/backbone_graph.py:
    69-70,273: weight and input cast to fp32)."""
    return np.asarray(x, np.float64) @ np.asarray(w, np.float64).T


def codebooks_head_ref(hidden, weight, cache_position=None) -> np.ndarray:
    """BreezeCodebooksHead.forward (models/breeze.py:597-612): position i of
    hidden [B, L, H] times weight[c] ([C, H, V]) with c = i when there is no
    cache position and c = cache_position[i] - 1 otherwise."""
    hidden = np.asarray(hidden, np.float64)
    weight = np.asarray(weight, np.float64)
    L = hidden.shape[1]
    idx = np.arange(L) if cache_position is None else np.asarray(cache_position).reshape(-1) - 1
    return np.stack([hidden[:, i, :] @ weight[idx[i]] for i in range(L)], axis=1)


def rel_err(out, ref) -> float:
    """bench_gemv.py:53: max|out - ref| / max|ref|."""
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(out - ref).max() / max(np.abs(ref).max(), 1e-30))


# ----------------------------------------------------------------------------
# synthetic inputs (seed, W ~ N(0,0.02), gamma = 1+N(0,0.1),
# x ~ N(0,1) bf16)
# ----------------------------------------------------------------------------


def synth(n: int, k: int, m: int, seed: int = 0):
    """W fp32 [N,K] ~ N(0, 0.02); gamma bf16 = 1 + N(0, 0.1); x bf16 ~ N(0,1).
    Returned as (W f32, gamma bf16 bits, x bf16 bits)."""
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    gamma = f32_to_bf16_bits(np.float32(1.0) + rng.standard_normal(k, dtype=np.float32) * np.float32(0.1))
    x = f32_to_bf16_bits(rng.standard_normal((m, k), dtype=np.float32))
    return w, gamma, x


# ----------------------------------------------------------------------------
# Row-block tiled layout (include/bz_gemv.h, BZ_W_*_TILED[_PAIRED])
# ----------------------------------------------------------------------------


def tiled_chunk_bytes(n_units: int, int4: bool) -> int:
    """Bytes of one 16-row block: n_units tiles of 1024 bytes, then the int4
    (s, z) pairs (64 bytes per unit) or the 16 fp32 row scales, padded to 128."""
    raw = n_units * 1024 + (n_units * 64 if int4 else 64)
    return (raw + 127) // 128 * 128


def tiled_row_pos(n_total: int, rows, paired: bool):
    """(block, row within block) of logical rows ``rows`` of an n_total-row
    tiled weight.  Paired: gate row r (r < n/2) -> block r//8, row r%8; up row
    r -> block (r-n/2)//8, row 8 + (r-n/2)%8."""
    r = np.asarray(rows, dtype=np.int64)
    if paired:
        h = n_total // 2
        rr = np.where(r < h, r, r - h)
        return rr // 8, rr % 8 + np.where(r < h, 0, 8)
    return r // 16, r % 16


def _tile(rows_bytes, unit_bytes_count, scale_bytes, int4: bool, paired: bool) -> np.ndarray:
    n = rows_bytes.shape[0]
    nu = unit_bytes_count
    chunk = tiled_chunk_bytes(nu, int4)
    blk, tr = tiled_row_pos(n, np.arange(n), paired)
    buf = np.zeros((n // 16) * chunk, dtype=np.uint8)
    base = blk[:, None, None] * chunk + np.arange(nu)[None, :, None] * 1024 + tr[:, None, None] * 64 \
        + np.arange(64)[None, None, :]
    buf[base] = rows_bytes.reshape(n, nu, 64)
    if int4:
        so = blk[:, None, None] * chunk + nu * 1024 + np.arange(nu)[None, :, None] * 64 + tr[:, None, None] * 4 \
            + np.arange(4)[None, None, :]
        buf[so] = scale_bytes  # [n, nu, 4]
    else:
        so = blk[:, None] * chunk + nu * 1024 + tr[:, None] * 4 + np.arange(4)[None, :]
        buf[so] = scale_bytes  # [n, 4]
    return buf


def tile_int4(packed, sz_bits, paired: bool = False) -> np.ndarray:
    """Row-major even-low nibbles uint8 [N, K/2] + scales_zeros bf16 bits
    [K/128, N, 2] (group 128) -> the BZ_W_INT4_TILED[_PAIRED] bytes."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    n, half = packed.shape
    nu = half // 64
    sz = np.ascontiguousarray(np.asarray(sz_bits, dtype=np.uint16).transpose(1, 0, 2))  # [N, NU, 2]
    return _tile(packed, nu, sz.view(np.uint8).reshape(n, nu, 4), True, paired)


def tile_fp8(codes, scale, paired: bool = False) -> np.ndarray:
    """Row-major e4m3 codes uint8 [N, K] + fp32 row scales [N] -> the
    BZ_W_FP8_TILED[_PAIRED] bytes."""
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    n, k = codes.shape
    sc = np.ascontiguousarray(np.asarray(scale, dtype=np.float32).reshape(n))
    return _tile(codes, k // 64, sc.view(np.uint8).reshape(n, 4), False, paired)


def _untile(buf, n: int, row_bytes: int, int4: bool, paired: bool):
    nu = row_bytes // 64
    chunk = tiled_chunk_bytes(nu, int4)
    buf = np.asarray(buf, dtype=np.uint8)
    blk, tr = tiled_row_pos(n, np.arange(n), paired)
    base = blk[:, None, None] * chunk + np.arange(nu)[None, :, None] * 1024 + tr[:, None, None] * 64 \
        + np.arange(64)[None, None, :]
    rows = buf[base].reshape(n, row_bytes)
    if int4:
        so = blk[:, None, None] * chunk + nu * 1024 + np.arange(nu)[None, :, None] * 64 + tr[:, None, None] * 4 \
            + np.arange(4)[None, None, :]
        sz = np.ascontiguousarray(buf[so]).view(np.uint16).reshape(n, nu, 2).transpose(1, 0, 2)
        return rows, np.ascontiguousarray(sz)
    so = blk[:, None] * chunk + nu * 1024 + tr[:, None] * 4 + np.arange(4)[None, :]
    return rows, np.ascontiguousarray(buf[so]).view(np.float32).reshape(n)


def untile_int4(buf, n: int, k: int, paired: bool = False):
    """Inverse of tile_int4: (packed uint8 [N, K/2], scales_zeros bits [K/128, N, 2])."""
    return _untile(buf, n, k // 2, True, paired)


def untile_fp8(buf, n: int, k: int, paired: bool = False):
    """Inverse of tile_fp8: (codes uint8 [N, K], scale fp32 [N])."""
    return _untile(buf, n, k, False, paired)
