"""Pins the oracle's SAM3 ViT glue: ggml_norm (sam3.cpp:1041-1051),
gelu_erf, the axial RoPE table (sam3.cpp:3559-3590; KATs of
tests/test_vit.cpp:182,192,218), RoPE application (sam3.cpp:3671-3710) and
ggml_win_part / win_unpart (sam3.cpp:3734,3788)."""
import math

import numpy as np
from scipy.special import erf


def test_norm(orc):
    x = orc.normal(7 * 1024, 0, 1).reshape(7, 1024) * 3 + 1.5
    y = np.empty_like(x)
    orc.lib().orc_norm_rows(x.ctypes.data, y.ctypes.data, 7, 1024, 1e-5)
    xd = x.astype(np.float64)
    ref = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-5)
    assert np.abs(y - ref).max() < 2e-6


def test_gelu_erf(orc):
    x = np.linspace(-8, 8, 10001, dtype=np.float32)
    y = np.empty_like(x)
    orc.lib().orc_gelu_erf(x.ctypes.data, y.ctypes.data, x.size)
    ref = 0.5 * x.astype(np.float64) * (1 + erf(x.astype(np.float64) / math.sqrt(2)))
    assert np.abs(y - ref).max() < 1e-5


def test_axial_cis_kat(orc):
    # window 24x24 scale 1 and global 72x72 scale 1/3, dim 64, theta 1e4, max diff < 1e-5
    for end, scale in ((24, 1.0), (72, 1.0 / 3.0)):
        n = end * end
        out = np.empty(n * 64, dtype=np.float32)
        orc.lib().orc_compute_axial_cis(out.ctypes.data, 64, end, end, 10000.0, scale)
        idx = np.arange(n)
        tx = (idx % end) * scale
        ty = (idx // end) * scale
        freqs = 1.0 / 10000.0 ** (np.arange(16) * 4 / 64)
        ax = tx[:, None] * freqs[None, :]
        ay = ty[:, None] * freqs[None, :]
        ref = np.concatenate([np.stack([np.cos(ax), np.sin(ax)], -1).reshape(n, 32),
                              np.stack([np.cos(ay), np.sin(ay)], -1).reshape(n, 32)], axis=1)
        assert np.abs(out.reshape(n, 64) - ref).max() < 1e-5


def test_rope_complex_multiply(orc):
    hd, n, rows = 64, 50, 3
    x = orc.normal(rows * n * hd, 0, 3).reshape(rows, n, hd)
    f = np.empty(n * hd, dtype=np.float32)
    orc.lib().orc_compute_axial_cis(f.ctypes.data, 64, 10, 5, 10000.0, 1.0)
    y = x.copy()
    orc.lib().orc_apply_rope(y.ctypes.data, f.ctypes.data, hd, n, rows)
    xc = x[..., 0::2].astype(np.float64) + 1j * x[..., 1::2]
    fc = f.reshape(n, 32, 2)
    fc = fc[..., 0].astype(np.float64) + 1j * fc[..., 1]
    ref = xc * fc[None]
    assert np.abs(y[..., 0::2] - ref.real).max() < 1e-5
    assert np.abs(y[..., 1::2] - ref.imag).max() < 1e-5


def test_win_part_unpart(orc):
    C, W, H, w = 8, 10, 7, 4
    x = orc.normal(C * W * H, 0, 5).reshape(H, W, C)
    npx, npy = 3, 2
    part = np.empty((npy * npx, w, w, C), dtype=np.float32)
    orc.lib().orc_win_part(x.ctypes.data, part.ctypes.data, C, W, H, w)
    pad = np.zeros((npy * w, npx * w, C), dtype=np.float32)
    pad[:H, :W] = x
    ref = pad.reshape(npy, w, npx, w, C).transpose(0, 2, 1, 3, 4).reshape(npy * npx, w, w, C)
    assert np.array_equal(part, ref)
    back = np.empty_like(x)
    orc.lib().orc_win_unpart(part.ctypes.data, back.ctypes.data, C, W, H, w)
    assert np.array_equal(back, x)
