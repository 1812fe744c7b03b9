"""GPU parity of the automatic launch choice over the tiled formats on a fixed,
seeded sample of shapes: every path the built-in rule and the static table
can pick for a tiled weight (the one-block and several-block streaming
kernels, the panel kernel over the whole K or over K slices, the tile kernel
for several rows with RMSNorm), with ragged row counts, both formats, paired
and plain weights, each epilogue and both output types, against the CPU
oracle on the same packed weights.

Bar: max|out-ref|/max|ref| <= 4e-3 against the same-rounding oracle (RMSNorm
folded as the kernels fold it), as for the fixed-shape tests.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import bz_oracle as O
from tests._util import Fp8Case, Int4Case, bf16_tensor, f32

pytestmark = pytest.mark.gpu

TIGHT = 4e-3

from breeze_amd import gemv as G  # noqa: E402


def _cases(n_cases: int = 36, seed: int = 2024):
    rng = np.random.default_rng(seed)
    ms = [1, 2, 3, 4, 5, 6, 7, 8, 9, 12, 16, 17, 24, 32, 33, 40]
    out = []
    for i in range(n_cases):
        fmt = "int4" if i % 2 == 0 else "fp8"
        unit = 128 if fmt == "int4" else 64
        paired = rng.random() < 0.3
        k = unit * int(rng.integers(1, 10240 // unit + 1))
        nblk = int(rng.integers(1, 700))
        while nblk * 16 * k > 6_000_000 and nblk > 1:  # keeps the oracle quick
            nblk //= 2
        n = 16 * nblk
        m = int(rng.choice(ms))
        norm = bool(rng.random() < 0.4)
        epi = G.EPI_SILU_GATE if paired else (G.EPI_RESIDUAL if rng.random() < 0.5 else G.EPI_NONE)
        out_f32 = bool(rng.random() < 0.25)
        out.append((fmt, paired, n, k, m, norm, epi, out_f32, 3000 + i))
    return out


# plus one case per path the sample might miss: the panel kernel over K
# slices (x above 128 KB; few row blocks), the tile kernel (several rows with
# RMSNorm), the several-block kernel over 5 blocks (more than 256 blocks)
CASES = _cases(96) + [
    ("int4", False, 1024, 8192, 24, False, G.EPI_RESIDUAL, False, 4001),
    ("fp8", False, 512, 10240, 12, False, G.EPI_NONE, True, 4002),
    ("int4", False, 2048, 2048, 33, True, G.EPI_RESIDUAL, False, 4003),
    ("int4", True, 20480, 256, 2, True, G.EPI_SILU_GATE, False, 4004),
]


@pytest.mark.parametrize("fmt,paired,n,k,m,norm,epi,out_f32,seed", CASES,
                         ids=[f"{c[0]}{'p' if c[1] else ''}-N{c[2]}-K{c[3]}-M{c[4]}-n{int(c[5])}-e{c[6]}-"
                              f"{'f32' if c[7] else 'bf16'}" for c in CASES])
def test_tiled_random_shapes_match_oracle(fmt, paired, n, k, m, norm, epi, out_f32, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    if fmt == "int4":
        c = Int4Case(w, 128, symmetric=True)
        wf = G.W_INT4_TILED_PAIRED if paired else G.W_INT4_TILED
        buf = G.pack_tiled(G.W_INT4_ZP, c.d_packed, k, wf, sc0=c.d_sz)
        w_eff = c.w_zp
    else:
        c = Fp8Case(w)
        wf = G.W_FP8_TILED_PAIRED if paired else G.W_FP8_TILED
        buf = G.pack_tiled(G.W_FP8, c.d_codes, k, wf, sc0=c.d_scale)
        w_eff = c.w_eff
    x_bits = O.f32_to_bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    g_bits = O.f32_to_bf16_bits((1 + 0.1 * rng.standard_normal(k)).astype(np.float32)) if norm else None
    n_out = n // 2 if epi == G.EPI_SILU_GATE else n
    r_bits = O.f32_to_bf16_bits(rng.standard_normal((m, n_out)).astype(np.float32)) if epi == G.EPI_RESIDUAL else None
    out = G.gemv(bf16_tensor(x_bits), buf, wf, n, gamma=bf16_tensor(g_bits) if norm else None, epilogue=epi,
                 residual=bf16_tensor(r_bits) if r_bits is not None else None,
                 out_dtype=torch.float32 if out_f32 else torch.bfloat16)
    assert out.shape == (m, n_out)
    xf = O.bf16_bits_to_f32(x_bits)
    xn = O.rmsnorm_folded(xf, O.bf16_bits_to_f32(g_bits)) if norm else xf
    ref = O.gemv_ref(xn, w_eff, epi, O.bf16_bits_to_f32(r_bits) if r_bits is not None else None)
    assert O.rel_err(f32(out), ref) <= TIGHT
