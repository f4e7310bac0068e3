"""Pins the oracle's SAM2 Hiera glue:
- ggml_gelu (tanh form) with ggml-cpu's fp16-table semantics (used by the
  Hiera MLP, sam3.cpp:4453), against the closed form in float64;
- sam2_window_partition / sam2_window_unpartition (sam3.cpp:4194-4281),
  against a numpy replay of the reference's own ggml reshape / permute / cont
  sequence (ggml ne [a, b, c, d] is numpy shape (d, c, b, a));
- sam2_maxpool_2d (sam3.cpp:4286-4296) against numpy.
"""
import math

import numpy as np
import pytest


def test_gelu_tanh_table(orc):
    # every finite half in (-10, 10), plus the clamps and off-grid inputs
    h = np.arange(65536, dtype=np.uint16).view(np.float16)
    h = h[np.isfinite(h)]
    x = h.astype(np.float32)
    y = np.empty_like(x)
    orc.lib().orc_gelu_tanh(x.ctypes.data, y.ctypes.data, x.size)
    xd = x.astype(np.float64)
    exact = 0.5 * xd * (1 + np.tanh(math.sqrt(2 / math.pi) * xd * (1 + 0.044715 * xd * xd)))
    inside = (x > -10) & (x < 10)
    # inside: the fp16 rounding of the fp32 evaluation -> within one half-ulp of exact
    # plus the fp32 evaluation error (bounded by 4 fp32 ulps of the larger terms)
    ulp16 = np.spacing(np.abs(exact[inside]).astype(np.float16)).astype(np.float64)
    assert (np.abs(y[inside] - exact[inside]) <= 0.5 * ulp16 + 4e-7 * np.abs(xd[inside]) + 1e-12).all()
    # every inside result is itself an fp16 value
    assert np.array_equal(y[inside], y[inside].astype(np.float16).astype(np.float32))
    assert (y[x <= -10] == 0).all()
    assert np.array_equal(y[x >= 10], x[x >= 10])
    # an input between halves uses the table entry of its fp16 rounding
    z = np.array([0.1000001, -1.23456, 3.33333], dtype=np.float32)
    yz = np.empty_like(z)
    orc.lib().orc_gelu_tanh(z.ctypes.data, yz.ctypes.data, z.size)
    zr = z.astype(np.float16).astype(np.float32)
    yr = np.empty_like(zr)
    orc.lib().orc_gelu_tanh(zr.ctypes.data, yr.ctypes.data, zr.size)
    assert np.array_equal(yz, yr)


def _ggml_window_partition(x, ws):
    """numpy replay of sam2_window_partition (sam3.cpp:4212-4232): x is a ggml
    tensor ne [C, W, H, B] held as numpy (B, H, W, C)."""
    B, H, W, C = x.shape
    Hp, Wp = -(-H // ws) * ws, -(-W // ws) * ws
    if Hp != H or Wp != W:                       # ggml_pad with zeros at the end of W and H
        x = np.pad(x, ((0, 0), (0, Hp - H), (0, Wp - W), (0, 0)))
    nWw, nWh = Wp // ws, Hp // ws
    r1 = x.reshape(B, Hp, nWw, C * ws)           # ggml reshape_4d [C*ws, nW_w, Hp, B]
    c1 = np.ascontiguousarray(r1.transpose(0, 2, 1, 3))  # permute(0,2,1,3) + cont -> [C*ws, Hp, nW_w, B]
    r2 = c1.reshape(nWw * B, nWh, ws, C * ws)    # [C*ws, ws, nW_h, nW_w*B]
    return r2.reshape(nWh * nWw * B, ws, ws, C)  # [C, ws, ws, nW*B]


def _ggml_window_unpartition(x, ws, Hp, Wp, H, W, B=1):
    """numpy replay of sam2_window_unpartition (sam3.cpp:4253-4281)."""
    C = x.shape[-1]
    nWh, nWw = Hp // ws, Wp // ws
    r1 = x.reshape(nWw * B, nWh, ws, C * ws)      # [C*ws, ws, nW_h, nW_w*B]
    r2 = r1.reshape(B, nWw, Hp, C * ws)           # [C*ws, Hp, nW_w, B]
    c1 = np.ascontiguousarray(r2.transpose(0, 2, 1, 3))  # [C*ws, nW_w, Hp, B]
    out = c1.reshape(B, Hp, Wp, C)                # [C, Wp, Hp, B]
    return np.ascontiguousarray(out[:, :H, :W, :])


@pytest.mark.parametrize("C,W,H,ws", [(3, 16, 16, 8), (5, 64, 64, 14), (2, 32, 32, 7), (4, 10, 6, 4)])
def test_hiera_window_partition(orc, C, W, H, ws):
    x = orc.normal(C * W * H, 0, 7).reshape(1, H, W, C)
    ref = _ggml_window_partition(x, ws)
    out = np.empty(ref.shape, dtype=np.float32)
    orc.lib().orc_hiera_win_part(x.ctypes.data, out.ctypes.data, C, W, H, ws)
    assert np.array_equal(out, ref)
    Hp, Wp = -(-H // ws) * ws, -(-W // ws) * ws
    back_ref = _ggml_window_unpartition(ref, ws, Hp, Wp, H, W)
    back = np.empty((H, W, C), dtype=np.float32)
    orc.lib().orc_hiera_win_unpart(np.ascontiguousarray(ref).ctypes.data, back.ctypes.data, C, W, H, ws)
    assert np.array_equal(back, back_ref[0])
    assert np.array_equal(back, x[0])


def test_maxpool2(orc):
    C, W, H, B = 3, 8, 6, 2
    x = orc.normal(B * H * W * C, 0, 8).reshape(B, H, W, C)
    out = np.empty((B, H // 2, W // 2, C), dtype=np.float32)
    orc.lib().orc_maxpool2(x.ctypes.data, out.ctypes.data, C, W, H, B)
    ref = x.reshape(B, H // 2, 2, W // 2, 2, C).max(axis=(2, 4))
    assert np.array_equal(out, ref)


def _tile(win, H, W):
    E, ws, _ = win.shape
    return np.tile(win, (1, H // ws + 1, W // ws + 1))[:, :H, :W]


@pytest.mark.parametrize("E,bh,bw,ws,H,W", [(96, 7, 7, 8, 256, 256), (8, 7, 7, 8, 64, 48), (4, 5, 9, 3, 12, 10)])
def test_sam2_pos_embed_vs_torch_bicubic(orc, E, bh, bw, ws, H, W):
    """sam2_bicubic_interpolate_cpu mirrors torch's bicubic upsampling
    (align_corners=False, A = -0.75, border-clamped taps): the oracle agrees
    with torch.nn.functional.interpolate to float rounding, plus the window
    table tiled modulo ws."""
    import torch
    rng = np.random.default_rng(E + H)
    bkg = rng.standard_normal((E, bh, bw)).astype(np.float32)
    win = rng.standard_normal((E, ws, ws)).astype(np.float32)
    got = orc.sam2_pos_embed(bkg, win, H, W)
    up = torch.nn.functional.interpolate(torch.from_numpy(bkg)[None], size=(H, W), mode="bicubic",
                                         align_corners=False)[0].numpy()
    ref = (up + _tile(win, H, W)).reshape(E, H * W).T
    assert np.abs(got - ref).max() <= 2e-5 * (np.abs(bkg).max() + np.abs(win).max())


def test_sam2_pos_embed_closed_forms(orc):
    """Equal sizes: every source coordinate is an integer, the taps weigh
    (0, 1, 0, 0) and the output is the input bit for bit.  A constant table
    stays constant (the four weights sum to 1).  A unit impulse at (3, 3) of a
    7x7 table upsampled 2x gives the separable kernel: source coordinate
    f = y/2 - 0.25, out(y, x) = w(f_y - 3) w(f_x - 3) with the Keys weights
    (a = -0.75) worked by hand: w(0.25) = 0.87890625, w(0.75) = 0.26171875,
    w(1.25) = -0.10546875, w(1.75) = -0.03515625, 0 beyond 2."""
    rng = np.random.default_rng(1)
    E, n = 6, 9
    bkg = rng.standard_normal((E, n, n)).astype(np.float32)
    zero = np.zeros((E, 1, 1), np.float32)
    got = orc.sam2_pos_embed(bkg, zero, n, n)
    assert np.array_equal(got, bkg.reshape(E, -1).T)
    const = np.full((E, 7, 7), 0.75, np.float32)
    got = orc.sam2_pos_embed(const, zero, 40, 24)
    assert np.abs(got - 0.75).max() <= 1e-6
    imp = np.zeros((1, 7, 7), np.float32)
    imp[0, 3, 3] = 1.0
    got = orc.sam2_pos_embed(imp, np.zeros((1, 1, 1), np.float32), 14, 14).reshape(14, 14)
    wtab = {0.25: 0.87890625, 0.75: 0.26171875, 1.25: -0.10546875, 1.75: -0.03515625}
    w1 = np.array([wtab.get(abs(y / 2 - 0.25 - 3), 0.0) for y in range(14)])
    assert np.count_nonzero(w1) == 8
    assert np.abs(got - np.outer(w1, w1)).max() <= 1e-7
