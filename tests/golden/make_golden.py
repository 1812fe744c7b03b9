"""Write the golden fixtures of the decode GEMV path (run from the repo root):

    python tests/golden/make_golden.py

The reference ships no vectors for this path (it has no automated test of
it), so the fixtures are produced by the CPU oracle (oracle/bz_oracle.py)
from fixed seeds, after the oracle itself has been pinned by
tests/test_oracle.py.  They freeze the quantizers' outputs, both nibble
orders, the scales_zeros layout, the dequantized weights and small GEMV
outputs, so a later change to the oracle or to the GPU path that moves a
single bit is caught.  Inputs are stored as raw bit patterns (bf16 as
uint16, fp8 as uint8).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import bz_oracle as O  # noqa: E402


def int4_case(seed: int, n: int, k: int, m: int, group: int, symmetric: bool) -> dict:
    w, gamma, x = O.synth(n, k, m, seed=seed)
    if symmetric:
        q, s, z = O.quantize_int4_sym(w, group)
        lo = (-8.0 * s).astype(np.float32)
    else:
        q, s, lo, z = O.quantize_int4_asym(w, group)
    sz = O.scales_zeros(s, z)
    s_bits, m_bits = O.f32_to_bf16_bits(s), O.f32_to_bf16_bits(lo)
    w_zp = O.dequant_int4_zp(q, sz, group)
    w_min = O.dequant_int4_min(q, s_bits, m_bits, group)
    xf, gf = O.bf16_bits_to_f32(x), O.bf16_bits_to_f32(gamma)
    xn = O.rmsnorm_f32(xf, gf)
    res = O.f32_to_bf16_bits(np.random.default_rng(seed + 100).standard_normal((m, n)).astype(np.float32))
    return {
        "w": w, "gamma": gamma, "x": x, "q": q, "s": s, "lo": lo, "z": z,
        "packed_even_low": O.pack_nibbles_even_low(q), "packed_odd_low": O.pack_nibbles_odd_low(q),
        "scales_zeros": sz, "scale_bits": s_bits, "min_bits": m_bits,
        "w_eff_zp": w_zp, "w_eff_min": w_min, "residual": res,
        "out_norm_none": O.gemv_ref(xn, w_zp).astype(np.float32),
        "out_norm_silu": O.gemv_ref(xn, w_zp, O.EPI_SILU).astype(np.float32),
        "out_plain_res": O.gemv_ref(xf, w_zp, O.EPI_RES, O.bf16_bits_to_f32(res)).astype(np.float32),
        "out_min_none": O.gemv_ref(xf, w_min).astype(np.float32),
        "meta": np.array([n, k, m, group, int(symmetric)], dtype=np.int64),
    }


def fp8_case(seed: int, n: int, k: int, m: int) -> dict:
    w, gamma, x = O.synth(n, k, m, seed=seed)
    codes, scale = O.quantize_fp8_linear(w)
    codes8, scale8 = O.pack_fp8(w)
    xf, gf = O.bf16_bits_to_f32(x), O.bf16_bits_to_f32(gamma)
    w_eff = O.dequant_fp8(codes, scale)
    return {
        "w": w, "gamma": gamma, "x": x, "codes": codes, "scale": scale, "codes_fused": codes8,
        "scale_fused": scale8, "w_eff": w_eff,
        "out_norm_none": O.gemv_ref(O.rmsnorm_f32(xf, gf), w_eff).astype(np.float32),
        "out_plain_silu": O.gemv_ref(xf, w_eff, O.EPI_SILU).astype(np.float32),
        "meta": np.array([n, k, m], dtype=np.int64),
    }


def main() -> None:
    cases = {
        "int4_asym_g128": int4_case(11, 48, 512, 2, 128, False),
        "int4_sym_g128": int4_case(12, 32, 384, 1, 128, True),
        "int4_asym_g32": int4_case(13, 24, 256, 3, 32, False),
        "fp8_row": fp8_case(14, 40, 256, 2),
    }
    for name, arrays in cases.items():
        np.savez_compressed(HERE / f"{name}.npz", **arrays)
    np.savez_compressed(HERE / "e4m3fn_table.npz", codes=np.arange(256, dtype=np.uint8),
                        values=O.e4m3fn_decode_table())
    print("wrote", ", ".join(sorted(cases)), "+ e4m3fn_table")


if __name__ == "__main__":
    main()
