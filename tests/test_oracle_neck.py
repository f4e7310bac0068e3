"""The neck oracle (oracle/neck.py) against torch's own convolution,
transposed convolution and max-pool in float64: the kernel layouts (ggml
memory order = torch's weight order), im2col's K order, padding, the
scatter of the transposed convolution and the pooling window are what these
fix; the f16 operand rounding is applied to both sides."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import neck


def _nchw(x, H, W):
    return torch.from_numpy(np.asarray(x, np.float64).reshape(H, W, -1).transpose(2, 0, 1).copy())[None]


def _tok(t):
    c = t.shape[1]
    return t[0].numpy().transpose(1, 2, 0).reshape(-1, c)


@pytest.mark.parametrize("Cin,Cout,k,s,H,W", [(16, 8, 2, 2, 5, 7), (8, 4, 3, 2, 4, 3), (6, 5, 2, 1, 3, 4)])
def test_conv_transpose_vs_torch(Cin, Cout, k, s, H, W):
    rng = np.random.default_rng(Cin * k + s)
    x = rng.standard_normal((H * W, Cin)).astype(np.float32)
    w = rng.standard_normal((Cin, Cout, k, k)).astype(np.float32)
    got = neck.conv_transpose_2d_p0(x, H, W, w, s)
    ref = F.conv_transpose2d(_nchw(neck.f16r(x), H, W), torch.from_numpy(neck.f16r(w).astype(np.float64)), stride=s)
    assert got.shape == (((H - 1) * s + k) * ((W - 1) * s + k), Cout)
    assert np.allclose(got, _tok(ref), rtol=0, atol=1e-12)
    assert np.all(neck.conv_transpose_2d_p0(x, H, W, w, s, absterm=True) >= np.abs(got) - 1e-12)
    rows = np.array([0, 5, got.shape[0] - 1, got.shape[0] // 2])
    assert np.allclose(neck.conv_transpose_2d_p0(x, H, W, w, s, rows=rows), got[rows], rtol=0, atol=1e-12)


@pytest.mark.parametrize("wtype", [neck.F32, neck.F16])
@pytest.mark.parametrize("Cin,Cout,k,s,p,H,W", [(12, 7, 1, 1, 0, 6, 5), (8, 6, 3, 1, 1, 7, 9), (5, 4, 2, 2, 0, 6, 8)])
def test_conv2d_vs_torch(wtype, Cin, Cout, k, s, p, H, W):
    rng = np.random.default_rng(Cin + 10 * k)
    x = rng.standard_normal((H * W, Cin)).astype(np.float32)
    w = rng.standard_normal((Cout, Cin, k, k)).astype(np.float32)
    if wtype == neck.F16:
        w = neck.f16r(w)
    got = neck.conv_2d(x, H, W, w, wtype, s, p)
    xin = neck.f16r(x) if wtype == neck.F16 else x
    ref = F.conv2d(_nchw(xin, H, W), torch.from_numpy(w.astype(np.float64)), stride=s, padding=p)
    assert np.allclose(got, _tok(ref), rtol=0, atol=1e-12)
    rows = np.array([0, 3, (ref.shape[2] * ref.shape[3]) - 1])
    assert np.allclose(neck.conv_2d(x, H, W, w, wtype, s, p, rows=rows), got[rows], rtol=0, atol=1e-12)


def test_maxpool_vs_torch():
    rng = np.random.default_rng(3)
    H, W, C = 6, 8, 5
    x = rng.standard_normal((H * W, C)).astype(np.float32)
    ref = F.max_pool2d(_nchw(x, H, W), 2, 2)
    assert np.array_equal(neck.maxpool2(x, H, W), _tok(ref).astype(np.float32))


def test_neck_shapes(orc):
    rng = np.random.default_rng(0)
    E, D, G = 16, 8, 6
    r = lambda *s: (rng.standard_normal(s) * 0.1).astype(np.float32)
    scales = [dict(deconv1_w=r(E, E // 2, 2, 2), deconv1_b=r(E // 2), deconv2_w=r(E // 2, D, 2, 2), deconv2_b=r(D),
                   conv1x1_w=r(D, D, 1, 1), conv1x1_b=r(D), conv3x3_w=r(D, D, 3, 3), conv3x3_b=r(D), wtype=neck.F32),
              dict(deconv1_w=r(E, E // 2, 2, 2), deconv1_b=r(E // 2), conv1x1_w=r(D, E // 2, 1, 1), conv1x1_b=r(D),
                   conv3x3_w=r(D, D, 3, 3), conv3x3_b=r(D), wtype=neck.F32)]
    scales += [dict(conv1x1_w=r(D, E, 1, 1), conv1x1_b=r(D), conv3x3_w=r(D, D, 3, 3), conv3x3_b=r(D), wtype=neck.F32)
               for _ in range(2)]
    outs = neck.sam3_neck(orc, r(G * G, E), G, scales)
    assert [o.shape for o in outs] == [(576, D), (144, D), (36, D), (9, D)]
    assert all(o.dtype == np.float32 and np.isfinite(o).all() for o in outs)
