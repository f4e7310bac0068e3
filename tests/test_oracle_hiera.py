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
