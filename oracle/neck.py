"""CPU restatement of sam3.cpp's SimpleFPN neck (sam3_build_neck_graph,
sam3.cpp:3867-3925) with ggml-cpu's convolution semantics.

TEST INFRASTRUCTURE ONLY: imported by tests/ (and nothing in the product).

Layouts.  Activations are token-major [H*W][C] float32: ggml [C, W, H], the
layout of the ViT output the neck reads and of the four maps it returns after
its final cont(permute(.., 1, 2, 0, 3)).  Kernels are numpy arrays in ggml
memory order: conv-transpose [Cin][Cout][kH][kW] (ggml ne [kW, kH, Cout,
Cin]), conv [Cout][Cin][kH][kW] (ggml ne [kW, kH, Cin, Cout]).

Arithmetic, per op, as ggml-cpu computes it:
- ggml_conv_transpose_2d_p0: the kernel is cast to F16 first
  (sam3_conv_transpose_weight, sam3.cpp:1087-1090) and the op converts its
  input to F16; each output is a sum of f16*f16 products over Cin.
- ggml_conv_2d (conv_2d_sk_p0 / conv_2d_s1_ph): im2col in the kernel's type
  (F32, or F16 with round-to-nearest-even of the activations), K ordered
  (ic, kh, kw), then MUL_MAT with f32 accumulation.
- ggml_pool_2d MAX 2x2 / 2: the window maximum.
- add_bias = ggml_add with the bias repeated: an f32 add; ggml_gelu_erf in f32.
Sums here run in float64 over the same rounded operands and are rounded to
f32 once per op; the reference's f32 summation order is not reproducible
(SIMD order), so comparisons use a bound relative to the sum of |terms|
(`absterm=True` returns that sum).
"""
from __future__ import annotations

import numpy as np

F32, F16 = 0, 1


def f16r(a: np.ndarray) -> np.ndarray:
    return np.asarray(a, dtype=np.float32).astype(np.float16).astype(np.float32)


def conv_transpose_2d_p0(x: np.ndarray, H: int, W: int, wk: np.ndarray, stride: int, rows=None,
                         absterm: bool = False) -> np.ndarray:
    """x [H*W][Cin]; wk [Cin][Cout][kH][kW] -> [OH*OW (or the rows given)][Cout]
    float64, OH = (H-1)*stride + kH.  Every (input pixel, tap) adds x·w to
    output pixel (y*stride + kh, x*stride + kw)."""
    Cin, Cout, kH, kW = wk.shape
    OH, OW = (H - 1) * stride + kH, (W - 1) * stride + kW
    xr = f16r(x).astype(np.float64).reshape(H, W, Cin)
    wr = f16r(wk).astype(np.float64)
    if absterm:
        xr, wr = np.abs(xr), np.abs(wr)
    if rows is not None:
        rows = np.asarray(rows)
        res = np.zeros((rows.size, Cout))
        for i, r in enumerate(rows):
            oy, ox = divmod(int(r), OW)
            for kh in range(kH):
                for kw in range(kW):
                    iy, ix = oy - kh, ox - kw
                    if iy % stride or ix % stride:
                        continue
                    iy, ix = iy // stride, ix // stride
                    if 0 <= iy < H and 0 <= ix < W:
                        res[i] += xr[iy, ix] @ wr[:, :, kh, kw]
        return res
    out = np.zeros((OH, OW, Cout))
    for kh in range(kH):
        for kw in range(kW):
            out[kh:kh + (H - 1) * stride + 1:stride, kw:kw + (W - 1) * stride + 1:stride] += xr @ wr[:, :, kh, kw]
    return out.reshape(OH * OW, Cout)


def im2col(x: np.ndarray, H: int, W: int, KH: int, KW: int, stride: int, pad: int, rows=None) -> np.ndarray:
    """ggml_im2col (2-D): [OH*OW (or the rows given)][Cin*KH*KW], K = (ic, kh, kw),
    zero outside the image."""
    Cin = x.shape[1]
    OH, OW = (H + 2 * pad - KH) // stride + 1, (W + 2 * pad - KW) // stride + 1
    xp = np.zeros((H + 2 * pad, W + 2 * pad, Cin), dtype=x.dtype)
    xp[pad:pad + H, pad:pad + W] = x.reshape(H, W, Cin)
    rows = np.arange(OH * OW) if rows is None else np.asarray(rows)
    oy, ox = rows // OW, rows % OW
    cols = np.empty((rows.size, Cin, KH, KW), dtype=x.dtype)
    for kh in range(KH):
        for kw in range(KW):
            cols[:, :, kh, kw] = xp[oy * stride + kh, ox * stride + kw]
    return cols.reshape(rows.size, Cin * KH * KW)


def conv_2d(x: np.ndarray, H: int, W: int, wk: np.ndarray, wtype: int, stride: int, pad: int, rows=None,
            absterm: bool = False) -> np.ndarray:
    """x [H*W][Cin]; wk [Cout][Cin][KH][KW] (float32, or float16 values when
    wtype is F16) -> [rows][Cout] float64."""
    Cout, Cin, KH, KW = wk.shape
    xa = f16r(x) if wtype == F16 else np.asarray(x, np.float32)
    wa = np.asarray(wk, np.float32).reshape(Cout, -1).astype(np.float64)
    cols = im2col(xa, H, W, KH, KW, stride, pad, rows).astype(np.float64)
    if absterm:
        cols, wa = np.abs(cols), np.abs(wa)
    return cols @ wa.T


def maxpool2(x: np.ndarray, H: int, W: int) -> np.ndarray:
    C = x.shape[1]
    v = np.asarray(x, np.float32).reshape(H // 2, 2, W // 2, 2, C)
    return v.max(axis=(1, 3)).reshape((H // 2) * (W // 2), C)


def add_bias(y: np.ndarray, b: np.ndarray) -> np.ndarray:
    return (np.asarray(y, np.float64).astype(np.float32) + np.asarray(b, np.float32)[None, :]).astype(np.float32)


def gelu_erf(orc, y: np.ndarray) -> np.ndarray:
    y = np.ascontiguousarray(y, dtype=np.float32)
    out = np.empty_like(y)
    orc.lib().orc_gelu_erf(orc._p(y), orc._p(out), y.size)
    return out


def sam3_neck(orc, x: np.ndarray, G: int, scales) -> list:
    """The four maps of sam3_build_neck_graph from the ViT output x [G*G][E].
    scales[i]: dict with the kernels (ggml memory order) and biases:
    'deconv1_w/b', 'deconv2_w/b' (scale 0), 'deconv1_w/b' (scale 1),
    'conv1x1_w/b', 'conv3x3_w/b' and 'wtype' (F32/F16 of the conv kernels)."""
    outs = []
    for i, s in enumerate(scales):
        H = W = G
        y = np.asarray(x, np.float32)
        if i == 0:
            y = add_bias(conv_transpose_2d_p0(y, H, W, s["deconv1_w"], 2), s["deconv1_b"])
            H, W = 2 * H, 2 * W
            y = gelu_erf(orc, y)
            y = add_bias(conv_transpose_2d_p0(y, H, W, s["deconv2_w"], 2), s["deconv2_b"])
            H, W = 2 * H, 2 * W
        elif i == 1:
            y = add_bias(conv_transpose_2d_p0(y, H, W, s["deconv1_w"], 2), s["deconv1_b"])
            H, W = 2 * H, 2 * W
        elif i == 3:
            y = maxpool2(y, H, W)
            H, W = H // 2, W // 2
        y = add_bias(conv_2d(y, H, W, s["conv1x1_w"], s["wtype"], 1, 0), s["conv1x1_b"])
        y = add_bias(conv_2d(y, H, W, s["conv3x3_w"], s["wtype"], 1, 1), s["conv3x3_b"])
        outs.append(y)
    return outs
