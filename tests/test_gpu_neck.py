"""SAM3 SimpleFPN neck on the GPU (mi355_sam3_neck and its node groups,
sam3_build_neck_graph sam3.cpp:3867-3925) against the neck oracle.

Bars, per op (conv-transpose + bias [+ GELU], conv 1x1 / 3x3 + bias):
|gpu - oracle| <= 1e-5 * sum|terms| + 4 ulp(|oracle|) -- the oracle sums the
same rounded operands (F16 for the conv-transpose and for F16 kernels) in
float64, so the bound covers f32 accumulation order and the f32 bias add;
after GELU the bound is scaled by 1.2 (|GELU'| < 1.13).  Max-pool is
bit-exact.  The full neck equals, bit for bit, the same node groups called
one by one, and matches the oracle's chained neck within 1e-4 of each map's
largest magnitude (intermediate F16 roundings may flip by one ulp between
f32 sums of different order).  Full SAM3 sizes (E = 1024, 72x72 grid, C1 =
512, D = 256) are checked per op on sampled output pixels, each op fed the
GPU's own input."""
import ctypes as C

import numpy as np
import pytest
import torch

from gpu_helpers import dev
from oracle import neck

pytestmark = pytest.mark.gpu


def kernel_tensor(mi, arr, wtype, ne):
    """arr in ggml memory order; ne the ggml shape."""
    if wtype == mi.F16:
        d = dev(np.ascontiguousarray(arr, np.float16).view(np.uint16))
    else:
        d = dev(np.ascontiguousarray(arr, np.float32))
    return mi.from_torch(d, wtype, list(ne))


def bound_ok(got, ref, absterm, scale=1.0):
    tol = scale * 1e-5 * absterm + 4 * np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    err = np.abs(got.astype(np.float64) - ref)
    return bool(np.all(err <= tol)), float((err / np.maximum(absterm, 1e-30)).max())


def rand(rng, shape, std=1.0):
    return (rng.standard_normal(shape) * std).astype(np.float32)


def run_deconv(mi, ctx, w, wtype, b, x, H, W, gelu):
    Cin, Cout = w.shape[0], w.shape[1]
    wt = kernel_tensor(mi, w, wtype, [2, 2, Cout, Cin])
    bd, xd = dev(b), dev(x)
    y = torch.full((4 * H * W, Cout), float("nan"), dtype=torch.float32, device="cuda")
    ctx.neck_deconv(wt, bd.data_ptr(), xd.data_ptr(), H, W, gelu, y.data_ptr())
    ctx.synchronize()
    return y.cpu().numpy()


def run_conv(mi, ctx, w, wtype, b, x, H, W):
    Cout, Cin, k, _ = w.shape
    wt = kernel_tensor(mi, w, wtype, [k, k, Cin, Cout])
    bd, xd = dev(b), dev(x)
    y = torch.full((H * W, Cout), float("nan"), dtype=torch.float32, device="cuda")
    ctx.neck_conv(wt, bd.data_ptr(), xd.data_ptr(), H, W, y.data_ptr())
    ctx.synchronize()
    return y.cpu().numpy()


def check_deconv(orc, got, w, b, x, H, W, gelu, rows=None):
    pre = neck.conv_transpose_2d_p0(x, H, W, w, 2, rows=rows)
    at = neck.conv_transpose_2d_p0(x, H, W, w, 2, rows=rows, absterm=True) + np.abs(b)[None, :]
    ref = neck.add_bias(pre, b)
    if gelu:
        ref = neck.gelu_erf(orc, ref)
    g = got if rows is None else got[rows]
    ok, worst = bound_ok(g, ref.astype(np.float64), at, 1.2 if gelu else 1.0)
    assert ok, f"deconv rel err {worst:.3e}"


def check_conv(got, w, wtype, b, x, H, W, rows=None):
    k = w.shape[2]
    pad = 1 if k == 3 else 0
    ref = neck.add_bias(neck.conv_2d(x, H, W, w, wtype, 1, pad, rows=rows), b)
    at = neck.conv_2d(x, H, W, w, wtype, 1, pad, rows=rows, absterm=True) + np.abs(b)[None, :]
    g = got if rows is None else got[rows]
    ok, worst = bound_ok(g, ref.astype(np.float64), at)
    assert ok, f"conv k={k} rel err {worst:.3e}"


@pytest.mark.parametrize("wtype", ["f32", "f16"])
@pytest.mark.parametrize("gelu", [False, True])
@pytest.mark.parametrize("Cin,Cout,H,W", [(64, 32, 6, 5), (96, 40, 3, 11), (48, 12, 7, 3)])
def test_neck_deconv(mi, ctx, orc, wtype, gelu, Cin, Cout, H, W):
    rng = np.random.default_rng(Cin + H)
    t = mi.F16 if wtype == "f16" else mi.F32
    w = rand(rng, (Cin, Cout, 2, 2), 0.05)
    if t == mi.F16:
        w = neck.f16r(w)
    b, x = rand(rng, Cout, 0.1), rand(rng, (H * W, Cin))
    got = run_deconv(mi, ctx, w, t, b, x, H, W, gelu)
    check_deconv(orc, got, w, b, x, H, W, gelu)


@pytest.mark.parametrize("wtype", ["f32", "f16"])
@pytest.mark.parametrize("k", [1, 3])
@pytest.mark.parametrize("Cin,Cout,H,W", [(64, 32, 9, 7), (256, 64, 5, 6), (40, 12, 4, 13)])
def test_neck_conv(mi, ctx, orc, wtype, k, Cin, Cout, H, W):
    rng = np.random.default_rng(Cin + 7 * k)
    t = mi.F16 if wtype == "f16" else mi.F32
    w = rand(rng, (Cout, Cin, k, k), 0.05)
    if t == mi.F16:
        w = neck.f16r(w)
    b, x = rand(rng, Cout, 0.1), rand(rng, (H * W, Cin))
    got = run_conv(mi, ctx, w, t, b, x, H, W)
    check_conv(got, w, t, b, x, H, W)


@pytest.mark.parametrize("wtype", ["f32", "f16"])
@pytest.mark.parametrize("k", [1, 3])
def test_neck_conv_split_unaligned_out(mi, ctx, orc, wtype, k):
    """A grid small enough for the K split (one 128-pixel tile, K = 9 * 256): with the output
    and bias 16-byte aligned the partial sums and the reduce run, with both offset by 4 bytes
    the single-pass kernel does; both within the per-op bar."""
    rng = np.random.default_rng(40 + k)
    t = mi.F16 if wtype == "f16" else mi.F32
    Cin, Cout, H, W = 256, 64, 6, 7
    w = rand(rng, (Cout, Cin, k, k), 0.05)
    if t == mi.F16:
        w = neck.f16r(w)
    b, x = rand(rng, Cout, 0.1), rand(rng, (H * W, Cin))
    wt = kernel_tensor(mi, w, t, [k, k, Cin, Cout])
    xd = dev(x)
    for off in (0, 1):
        bbuf = torch.zeros(Cout + 4, dtype=torch.float32, device="cuda")
        bbuf[off:off + Cout] = torch.from_numpy(b).cuda()
        ybuf = torch.full((H * W * Cout + 4,), float("nan"), dtype=torch.float32, device="cuda")
        ctx.neck_conv(wt, bbuf.data_ptr() + 4 * off, xd.data_ptr(), H, W, ybuf.data_ptr() + 4 * off)
        ctx.synchronize()
        got = ybuf[off:off + H * W * Cout].cpu().numpy().reshape(H * W, Cout)
        check_conv(got, w, t, b, x, H, W)


@pytest.mark.parametrize("wtype", ["f32", "f16"])
def test_neck_conv3x3_unaligned_map(mi, orc, wtype):
    """A 3x3 over a map whose rows are not 16-byte aligned takes im2col + MUL_MAT;
    its scratch is sized for the columns (P * 9 * Cin), not for the repacked
    kernel, in a fresh context whose neck scratch has not grown before."""
    rng = np.random.default_rng(77)
    Cout, Cin, H, W = 32, 64, 17, 15
    t = mi.F16 if wtype == "f16" else mi.F32
    w = rand(rng, (Cout, Cin, 3, 3), 0.05)
    if t == mi.F16:
        w = neck.f16r(w)
    b, x = rand(rng, Cout, 0.1), rand(rng, (H * W, Cin))
    c = mi.Context(0)
    try:
        wt = kernel_tensor(mi, w, t, [3, 3, Cin, Cout])
        bd = dev(b)
        xd = torch.zeros(H * W * Cin + 1, dtype=torch.float32, device="cuda")
        xd[1:] = torch.from_numpy(x.reshape(-1)).cuda()
        y = torch.full((H * W, Cout), float("nan"), dtype=torch.float32, device="cuda")
        c.neck_conv(wt, bd.data_ptr(), xd.data_ptr() + 4, H, W, y.data_ptr())
        c.synchronize()
        got = y.cpu().numpy()
    finally:
        c.close()
    check_conv(got, w, t, b, x, H, W)


def test_neck_maxpool(mi, ctx):
    rng = np.random.default_rng(2)
    H, W, Cc = 10, 6, 12
    x = rand(rng, (H * W, Cc))
    xd = dev(x)
    y = torch.full((H * W // 4, Cc), float("nan"), dtype=torch.float32, device="cuda")
    ctx.neck_maxpool(xd.data_ptr(), H, W, Cc, y.data_ptr())
    ctx.synchronize()
    assert np.array_equal(y.cpu().numpy(), neck.maxpool2(x, H, W))


def _scales(mi, rng, E, C1, D, wt):
    f16 = wt == mi.F16

    def kw(shape, std=0.05):
        a = rand(rng, shape, std)
        return neck.f16r(a) if f16 else a

    sc = [dict(deconv1_w=kw((E, C1, 2, 2)), deconv1_b=rand(rng, C1, 0.1), deconv2_w=kw((C1, D, 2, 2)),
               deconv2_b=rand(rng, D, 0.1), conv1x1_w=kw((D, D, 1, 1)), conv1x1_b=rand(rng, D, 0.1),
               conv3x3_w=kw((D, D, 3, 3), 0.03), conv3x3_b=rand(rng, D, 0.1)),
          dict(deconv1_w=kw((E, C1, 2, 2)), deconv1_b=rand(rng, C1, 0.1), conv1x1_w=kw((D, C1, 1, 1)),
               conv1x1_b=rand(rng, D, 0.1), conv3x3_w=kw((D, D, 3, 3), 0.03), conv3x3_b=rand(rng, D, 0.1))]
    sc += [dict(conv1x1_w=kw((D, E, 1, 1)), conv1x1_b=rand(rng, D, 0.1), conv3x3_w=kw((D, D, 3, 3), 0.03),
                conv3x3_b=rand(rng, D, 0.1)) for _ in range(2)]
    for s in sc:
        s["wtype"] = wt
    return sc


def _device_scales(mi, sc):
    keep, out = [], []
    for s in sc:
        d = {}
        for f in ("deconv1", "deconv2", "conv1x1", "conv3x3"):
            if f + "_w" not in s:
                continue
            w = s[f + "_w"]
            ne = [2, 2, w.shape[1], w.shape[0]] if f.startswith("deconv") else [w.shape[2], w.shape[3], w.shape[1],
                                                                                 w.shape[0]]
            t = kernel_tensor(mi, w, s["wtype"], ne)
            bd = dev(s[f + "_b"])
            keep += [t, bd]
            d[f + "_w"], d[f + "_b"] = t, bd.data_ptr()
        out.append(d)
    return out, keep


def _run_neck(mi, ctx, x, E, G, dsc, D):
    xd = dev(x)
    sizes = [16 * G * G, 4 * G * G, G * G, G * G // 4]
    outs = [torch.full((n, D), float("nan"), dtype=torch.float32, device="cuda") for n in sizes]
    ctx.sam3_neck(xd.data_ptr(), E, G, dsc, [o.data_ptr() for o in outs])
    ctx.synchronize()
    return [o.cpu().numpy() for o in outs]


@pytest.mark.parametrize("wtype", ["f32", "f16"])
def test_sam3_neck_small(mi, ctx, orc, wtype):
    rng = np.random.default_rng(11)
    E, C1, D, G = 64, 32, 32, 8
    wt = mi.F16 if wtype == "f16" else mi.F32
    sc = _scales(mi, rng, E, C1, D, wt)
    x = rand(rng, (G * G, E))
    dsc, keep = _device_scales(mi, sc)
    got = _run_neck(mi, ctx, x, E, G, dsc, D)
    ref = neck.sam3_neck(orc, x, G, sc)
    for i, (g, r) in enumerate(zip(got, ref)):
        assert g.shape == r.shape
        assert np.abs(g - r).max() <= 1e-4 * np.abs(r).max(), f"scale {i}"
    # the same node groups one by one: bit-identical
    s0 = sc[0]
    a = run_deconv(mi, ctx, s0["deconv1_w"], wt, s0["deconv1_b"], x, G, G, True)
    a = run_deconv(mi, ctx, s0["deconv2_w"], wt, s0["deconv2_b"], a, 2 * G, 2 * G, False)
    a = run_conv(mi, ctx, s0["conv1x1_w"], wt, s0["conv1x1_b"], a, 4 * G, 4 * G)
    a = run_conv(mi, ctx, s0["conv3x3_w"], wt, s0["conv3x3_b"], a, 4 * G, 4 * G)
    assert np.array_equal(a, got[0])


@pytest.mark.parametrize("wtype", ["f32", "f16"])
def test_sam3_neck_full_size_per_op(mi, ctx, orc, wtype):
    """E = 1024 at 72x72 (SAM3 at 1008^2), C1 = 512, D = 256: every op of
    scales 0 and 3 on sampled pixels, fed the GPU's own input; the fused neck
    equals the ops composed."""
    rng = np.random.default_rng(5)
    E, C1, D, G = 1024, 512, 256, 72
    wt = mi.F16 if wtype == "f16" else mi.F32
    sc = _scales(mi, rng, E, C1, D, wt)
    x = rand(rng, (G * G, E))
    pick = lambda n: np.unique(np.concatenate([[0, n - 1], rng.choice(n, 96, replace=False)]))
    s0 = sc[0]
    a = run_deconv(mi, ctx, s0["deconv1_w"], wt, s0["deconv1_b"], x, G, G, True)
    check_deconv(orc, a, s0["deconv1_w"], s0["deconv1_b"], x, G, G, True, rows=pick(a.shape[0]))
    b = run_deconv(mi, ctx, s0["deconv2_w"], wt, s0["deconv2_b"], a, 2 * G, 2 * G, False)
    check_deconv(orc, b, s0["deconv2_w"], s0["deconv2_b"], a, 2 * G, 2 * G, False, rows=pick(b.shape[0]))
    c = run_conv(mi, ctx, s0["conv1x1_w"], wt, s0["conv1x1_b"], b, 4 * G, 4 * G)
    check_conv(c, s0["conv1x1_w"], wt, s0["conv1x1_b"], b, 4 * G, 4 * G, rows=pick(c.shape[0]))
    d = run_conv(mi, ctx, s0["conv3x3_w"], wt, s0["conv3x3_b"], c, 4 * G, 4 * G)
    check_conv(d, s0["conv3x3_w"], wt, s0["conv3x3_b"], c, 4 * G, 4 * G, rows=pick(d.shape[0]))
    s3 = sc[3]
    xd = dev(x)
    p = torch.empty((G * G // 4, E), dtype=torch.float32, device="cuda")
    ctx.neck_maxpool(xd.data_ptr(), G, G, E, p.data_ptr())
    ctx.synchronize()
    pn = p.cpu().numpy()
    assert np.array_equal(pn, neck.maxpool2(x, G, G))
    e = run_conv(mi, ctx, s3["conv1x1_w"], wt, s3["conv1x1_b"], pn, G // 2, G // 2)
    check_conv(e, s3["conv1x1_w"], wt, s3["conv1x1_b"], pn, G // 2, G // 2)
    f = run_conv(mi, ctx, s3["conv3x3_w"], wt, s3["conv3x3_b"], e, G // 2, G // 2)
    check_conv(f, s3["conv3x3_w"], wt, s3["conv3x3_b"], e, G // 2, G // 2)
    dsc, keep = _device_scales(mi, sc)
    got = _run_neck(mi, ctx, x, E, G, dsc, D)
    assert np.array_equal(got[0], d)
    assert np.array_equal(got[3], f)
    assert all(np.isfinite(g).all() for g in got)


@pytest.mark.parametrize("wtype", ["f32", "f16"])
def test_neck_random_shapes(mi, ctx, orc, wtype):
    """Seeded random conv / conv-transpose shapes against the per-op bars: map
    sizes ragged against the 128-pixel tiles, channel counts on both sides of
    the implicit-GEMM condition (Cin % 32 == 0), with and without GELU."""
    rng = np.random.default_rng(77 if wtype == "f32" else 78)
    t = mi.F16 if wtype == "f16" else mi.F32
    for i in range(10):
        H, W = int(rng.integers(1, 40)), int(rng.integers(1, 40))
        Cin = int(rng.choice([32, 64, 96, 20, 44]))
        Cout = 4 * int(rng.integers(1, 24))
        k = int(rng.choice([1, 3]))
        w = rand(rng, (Cout, Cin, k, k), 0.05)
        if t == mi.F16:
            w = neck.f16r(w)
        b, x = rand(rng, Cout, 0.1), rand(rng, (H * W, Cin))
        check_conv(run_conv(mi, ctx, w, t, b, x, H, W), w, t, b, x, H, W)
        wd = rand(rng, (Cin, Cout, 2, 2), 0.05)
        if t == mi.F16:
            wd = neck.f16r(wd)
        gelu = bool(i % 2)
        check_deconv(orc, run_deconv(mi, ctx, wd, t, b, x, H, W, gelu), wd, b, x, H, W, gelu)
