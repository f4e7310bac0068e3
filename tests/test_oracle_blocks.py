"""The oracle block compositions of tests/block_refs.py evaluated on a subset
of query rows equal the full compositions on those rows bit for bit (every
node is row-local after the attention, and the attention of one query does
not depend on the other queries), so the full-size GPU tests may sample
rows.  Also pins the window-order row map against ggml_win_part /
ggml_win_unpart."""
import types

import numpy as np
import pytest

from block_refs import axial_cis, hiera_block_ref, vit_block_ref, vit_block_rows, win_part, win_rows, win_unpart


def _vit_weights(orc, t, E, MLP, seed):
    shapes = {"qkv": (3 * E, E), "proj": (E, E), "fc1": (MLP, E), "fc2": (E, MLP)}
    host = {}
    for i, (name, (N, K)) in enumerate(shapes.items()):
        w = orc.normal(N * K, seed, 10 + i, std=0.02).reshape(N, K)
        host[name] = (orc.quantize_weights(t, w), N, K)
    vec = {}
    for i, (name, n, s, m) in enumerate([("norm1_w", E, 0.2, 1.0), ("norm1_b", E, 0.1, 0.0), ("qkv_b", 3 * E, 0.05, 0.0),
                                          ("proj_b", E, 0.05, 0.0), ("norm2_w", E, 0.2, 1.0), ("norm2_b", E, 0.1, 0.0),
                                          ("fc1_b", MLP, 0.05, 0.0), ("fc2_b", E, 0.05, 0.0)]):
        vec[name] = orc.normal(n, seed, 20 + i) * np.float32(s) + np.float32(m)
    return host, vec


def test_win_rows_matches_win_part(orc):
    grid, ws, E = 12, 4, 8
    x = orc.normal(grid * grid * E, 3, 1).reshape(grid * grid, E)
    perm = win_rows(orc, grid, ws)
    assert sorted(perm.tolist()) == list(range(grid * grid))
    assert np.array_equal(win_part(orc, x, grid, ws), x[perm])
    assert np.array_equal(win_unpart(orc, x[perm], grid, ws), x)


@pytest.mark.parametrize("ws", [0, 4])
@pytest.mark.parametrize("f16_attn", [False, True])
def test_vit_rows_equal_full(orc, ws, f16_attn):
    t = orc.Q8_0
    E, NH, MLP, grid = 64, 2, 128, 8
    host, vec = _vit_weights(orc, t, E, MLP, seed=5)
    x = orc.normal(grid * grid * E, 6, 1).reshape(grid * grid, E)
    freqs = axial_cis(orc, E // NH, ws or grid, 1.0 if ws else 0.5)
    full = vit_block_ref(orc, t, x, host, vec, E, NH, MLP, grid, ws, freqs, f16_attn)
    N = ws * ws if ws else grid * grid
    qsel = np.array([0, 3, N // 2, N - 1])
    rows, out = vit_block_rows(orc, t, x, host, vec, E, NH, MLP, grid, ws, freqs, f16_attn, qsel=qsel)
    assert len(rows) == len(qsel) * (grid * grid // N)
    assert np.array_equal(out, full[rows])


@pytest.mark.parametrize("f16_attn", [False, True])
def test_hiera_global_rows_equal_full(orc, f16_attn):
    t = orc.Q4_0
    C_, NH, S = 64, 2, 8
    info = types.SimpleNamespace(dim_in=C_, dim_out=C_, num_heads=NH, window_size=0, q_stride=0)
    shapes = {"qkv": (3 * C_, C_), "proj": (C_, C_), "fc1": (4 * C_, C_), "fc2": (C_, 4 * C_)}
    host = {n: (orc.quantize_weights(t, orc.normal(N * K, 7, 30 + i, std=0.05).reshape(N, K)), N, K)
            for i, (n, (N, K)) in enumerate(shapes.items())}
    vec = {n: orc.normal(c, 7, 50 + i) * np.float32(0.1) + np.float32(m)
           for i, (n, c, m) in enumerate([("norm1_w", C_, 1.0), ("norm1_b", C_, 0.0), ("qkv_b", 3 * C_, 0.0),
                                         ("proj_b", C_, 0.0), ("norm2_w", C_, 1.0), ("norm2_b", C_, 0.0),
                                         ("fc1_b", 4 * C_, 0.0), ("fc2_b", C_, 0.0)])}
    x = orc.normal(S * S * C_, 8, 1).reshape(S * S, C_)
    rows_all, full = hiera_block_ref(orc, t, x, info, host, vec, S, f16_attn)
    assert np.array_equal(rows_all, np.arange(S * S))
    qsel = np.array([1, 9, 40, 63])
    rows, out = hiera_block_ref(orc, t, x, info, host, vec, S, f16_attn, qsel=qsel)
    assert np.array_equal(rows, qsel)
    assert np.array_equal(out, full[qsel])
