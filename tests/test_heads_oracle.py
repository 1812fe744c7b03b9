"""Pins of the fp32 head restatements (CPU only)."""

from __future__ import annotations

import numpy as np
import torch

from oracle import bz_oracle as O


def test_linear_f32_matches_torch_float64():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 64)).astype(np.float32)
    w = rng.standard_normal((37, 64)).astype(np.float32)
    ref = torch.nn.functional.linear(torch.from_numpy(x).double(), torch.from_numpy(w).double()).numpy()
    np.testing.assert_allclose(O.linear_f32_ref(x, w), ref, rtol=1e-12)


def test_codebooks_head_matches_per_codebook_linear():
    rng = np.random.default_rng(1)
    C, H, V, B, L = 5, 32, 19, 2, 3
    weight = rng.standard_normal((C, H, V)).astype(np.float32)
    hidden = rng.standard_normal((B, L, H)).astype(np.float32)
    got = O.codebooks_head_ref(hidden, weight)
    for i in range(L):
        ref = torch.nn.functional.linear(torch.from_numpy(hidden[:, i]).double(),
                                         torch.from_numpy(weight[i]).double().T).numpy()
        np.testing.assert_allclose(got[:, i], ref, rtol=1e-12)


def test_codebook_selection_follows_cache_position():
    """weight[c] maps hidden unit 0 to vocab entry c only: the argmax of each
    output names the codebook that was used."""
    C, H, V = 6, 4, 8
    weight = np.zeros((C, H, V))
    for c in range(C):
        weight[c, 0, c] = 1.0
    hidden = np.zeros((1, 3, H))
    hidden[:, :, 0] = 1.0
    assert list(O.codebooks_head_ref(hidden, weight).argmax(-1)[0]) == [0, 1, 2]
    assert list(O.codebooks_head_ref(hidden, weight, np.array([4, 2, 6])).argmax(-1)[0]) == [3, 1, 5]
