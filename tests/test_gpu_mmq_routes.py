"""The int8 MUL_MAT routes: mi355_context_set_mmq_kernel(MI355_MMQ_INT8)
(one-byte activation quants, weights repacked into int8 rows with separate
scale arrays on each call, exact int32 block sums on v_mfma_i32_32x32x32_i8),
the default MI355_MMQ_AUTO, and weights prepared once by mi355_weight_prepare
(the int8 kernel without the per-call repack).

Bars:
  * block sums: bit-exact against numpy int64 dot products of the oracle's
    quants (mi355_mul_mat_block_dots on each route);
  * outputs: |gpu - oracle| <= 1e-5 * absterm (as every quantized mul_mat),
    and bit-identical to the MI355_MMQ_F16 route on the same operands: both
    combine acc = fma(isum, d_a * d_w, acc) in block order, so any difference
    is a defect of one of them.
Shapes: the four SAM3 ViT linears at 5184 tokens, ragged M / N, an odd block
count (K = 96, 4736 = 148 blocks), and GEMMs small enough to take split-K."""
import numpy as np
import pytest
import torch

from gpu_helpers import absterm, dev, rel_err

pytestmark = pytest.mark.gpu


ROUTES = ["int8", "auto", "prepared"]


def _kernel(mi, route):
    return {"f16": mi.MMQ_F16, "int8": mi.MMQ_INT8, "auto": mi.MMQ_AUTO, "prepared": mi.MMQ_AUTO}[route]


def _prepare(mi, ctx, wt):
    """The prepared form of wt in a fresh 256-byte aligned device buffer."""
    n = mi.weight_prepared_nbytes(wt)
    assert n > 0
    buf = torch.full((n + 256,), 0xAB, dtype=torch.uint8, device="cuda")
    off = (-buf.data_ptr()) % 256
    pt = ctx.weight_prepare(wt, buf.data_ptr() + off, n)
    pt._keep = (buf, wt._keep)
    return pt


def _weights(mi, ctx, wq, t, K, N, route):
    wt = mi.from_torch(dev(wq.view(np.uint8)), t, [K, N])
    return _prepare(mi, ctx, wt) if route == "prepared" else wt


def _run(mi, ctx, wq, t, K, N, x, route):
    M = x.shape[0]
    s0, xd = _weights(mi, ctx, wq, t, K, N, route), dev(x)
    dst = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    ctx.set_mmq_kernel(_kernel(mi, route))
    try:
        ctx.mul_mat(s0, mi.from_torch(xd, mi.F32, [K, M]), mi.from_torch(dst, mi.F32, [N, M]))
        ctx.synchronize()
    finally:
        ctx.set_mmq_kernel(mi.MMQ_AUTO)
    return dst


@pytest.mark.parametrize("route", ROUTES)
@pytest.mark.parametrize("tname", ["q8_0", "q4_0", "q4_1"])
@pytest.mark.parametrize("M,N,K", [(5184, 3072, 1024), (5184, 1024, 1024), (5184, 4736, 1024), (5184, 1024, 4736),
                                   (77, 65, 96), (300, 200, 1024), (33, 130, 4736), (1000, 96, 160), (129, 257, 64)])
def test_route_bit_identical(mi, ctx, orc, route, tname, M, N, K):
    t = orc.NAME_TYPE[tname]
    print(f"{route} route {tname} M={M} N={N} K={K}", flush=True)
    w = orc.normal(N * K, seed=M + N, stream=1, std=0.02).reshape(N, K)
    x = orc.normal(M * K, seed=M + N, stream=2).reshape(M, K)
    wq = orc.quantize_weights(t, w)
    ref16 = _run(mi, ctx, wq, t, K, N, x, "f16")
    got8 = _run(mi, ctx, wq, t, K, N, x, route)
    assert torch.isfinite(got8).all()
    assert torch.equal(got8, ref16), f"max diff {(got8 - ref16).abs().max().item():.3e}"
    rows = np.arange(M) if M <= 300 else np.linspace(0, M - 1, 97).astype(int)
    vt = orc.VEC_DOT_TYPE[t]
    ref = orc.mul_mat(wq, t, K, N, x[rows][None, None])[0, 0]
    e = rel_err(got8.cpu().numpy()[rows], ref, absterm(orc, t, wq, K, orc.from_float(vt, x[rows])))
    assert e <= 1e-5, f"rel err {e:.3e}"


@pytest.mark.parametrize("route", ["int8", "prepared"])
@pytest.mark.parametrize("tname", ["q8_0", "q4_0", "q4_1"])
@pytest.mark.parametrize("M,N,K", [(65536, 288, 96), (5000, 100, 64), (4097, 36, 128), (8192, 384, 32),
                                   (16384, 192, 96), (4096, 576, 96), (4100, 33, 96)])
def test_route_skinny_bit_identical(mi, ctx, orc, route, tname, M, N, K):
    """K <= 128 at M >= 4096 on the int8 routes runs on the skinny int8 kernel (N % 4 == 0;
    N = 33 stays tiled): bit-identical to the tiled int8 kernel (the skinny switch off) and
    to the fp16 route, ragged M and N included."""
    t = orc.NAME_TYPE[tname]
    print(f"{route} skinny {tname} M={M} N={N} K={K}", flush=True)
    w = orc.normal(N * K, seed=N + K, stream=1, std=0.02).reshape(N, K)
    x = orc.normal(M * K, seed=N + K, stream=2).reshape(M, K)
    wq = orc.quantize_weights(t, w)
    got = _run(mi, ctx, wq, t, K, N, x, route)
    ctx.set_skinny(False)
    try:
        tiled = _run(mi, ctx, wq, t, K, N, x, route)
    finally:
        ctx.set_skinny(True)
    ref16 = _run(mi, ctx, wq, t, K, N, x, "f16")
    assert torch.isfinite(got).all()
    assert torch.equal(got, tiled), f"max diff {(got - tiled).abs().max().item():.3e}"
    assert torch.equal(got, ref16), f"max diff {(got - ref16).abs().max().item():.3e}"


@pytest.mark.parametrize("route", ROUTES)
@pytest.mark.parametrize("tname", ["q8_0", "q4_0", "q4_1"])
@pytest.mark.parametrize("K", [96, 1024])
def test_route_block_dots_bit_exact(mi, ctx, orc, route, tname, K):
    t = orc.NAME_TYPE[tname]
    M, N = 70, 45
    w = orc.normal(N * K, seed=4, stream=1, std=0.02).reshape(N, K)
    x = orc.normal(M * K, seed=4, stream=2).reshape(M, K)
    wq = orc.quantize_weights(t, w)
    nb = K // 32
    isums = torch.zeros(M * N * nb, dtype=torch.int32, device="cuda")
    s0 = _weights(mi, ctx, wq, t, K, N, route)
    ctx.set_mmq_kernel(_kernel(mi, route))
    try:
        ctx.mul_mat_block_dots(s0, mi.from_torch(dev(x), mi.F32, [K, M]), isums.data_ptr())
        ctx.synchronize()
    finally:
        ctx.set_mmq_kernel(mi.MMQ_AUTO)
    got = isums.cpu().numpy().reshape(M, N, nb)
    wv, _, _ = orc.decode_blocks(t, wq, K)
    xv, _, _ = orc.decode_blocks(orc.VEC_DOT_TYPE[t], orc.from_float(orc.VEC_DOT_TYPE[t], x), K)
    ref = np.einsum("mbj,nbj->mnb", xv.reshape(M, nb, 32).astype(np.int64), wv.reshape(N, nb, 32).astype(np.int64))
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("route", ROUTES)
def test_route_integer_exact(mi, ctx, orc, route):
    """Unit scales (d_a = d_w = 1) make the result an exact integer: each
    route must return sum_b isum_b bit for bit, with |isum| near the int8
    extremes (-127..127 on both sides)."""
    M, N, K = 96, 80, 1024
    rng = np.random.default_rng(12)
    x = rng.integers(-127, 128, size=(M, K)).astype(np.float32)
    x.reshape(M, K // 32, 32)[:, :, 5] = 127.0
    q = rng.integers(-127, 128, size=(N, K)).astype(np.int8)
    wq = np.zeros((N, K // 32, 34), dtype=np.uint8)
    wq[:, :, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    wq[:, :, 2:] = q.reshape(N, K // 32, 32).view(np.uint8)
    out = _run(mi, ctx, wq.reshape(N, -1), orc.Q8_0, K, N, x, route).cpu().numpy()
    exact = x.astype(np.int64) @ q.astype(np.int64).T
    assert np.array_equal(out, exact.astype(np.float32))


@pytest.mark.parametrize("tname", ["q8_0", "q4_0", "q4_1"])
def test_prepared_layout_and_rejections(mi, ctx, orc, tname):
    """Prepared-weight sizes (quants, then fp16 d, then Q4_1's fp16 m, each
    part 256-byte aligned), the no-allocation entry point on a prepared
    weight, and the calls that must refuse one."""
    t = orc.NAME_TYPE[tname]
    M, N, K = 200, 150, 96 + 32  # 4 blocks per row
    w = orc.normal(N * K, seed=9, stream=1, std=0.02).reshape(N, K)
    wq = orc.quantize_weights(t, w)
    wt = mi.from_torch(dev(wq.view(np.uint8)), t, [K, N])
    al = lambda v: (v + 255) // 256 * 256
    dp = 4
    want = al(N * K) + al(N * dp * 2) * (2 if tname == "q4_1" else 1)
    assert mi.weight_prepared_nbytes(wt) == want
    pt = _prepare(mi, ctx, wt)
    assert pt.layout == mi.LAYOUT_INT8 and list(pt.ne) == [K, N, 1, 1]
    assert mi.lib().mi355_tensor_nbytes(mi.C.byref(pt)) == want
    # mul_mat and mul_mat_noalloc on the prepared weight: the raw weight's bits
    x = dev(orc.normal(M * K, seed=9, stream=2).reshape(M, K))
    outs = [torch.full((M, N), float("nan"), device="cuda") for _ in range(3)]
    ctx.mul_mat(wt, mi.from_torch(x, mi.F32, [K, M]), mi.from_torch(outs[0], mi.F32, [N, M]))
    ctx.mul_mat(pt, mi.from_torch(x, mi.F32, [K, M]), mi.from_torch(outs[1], mi.F32, [N, M]))
    ctx.mul_mat_noalloc(pt, mi.from_torch(x, mi.F32, [K, M]), mi.from_torch(outs[2], mi.F32, [N, M]))
    ctx.synchronize()
    assert torch.equal(outs[1], outs[0]) and torch.equal(outs[2], outs[0])

    def status(fn):
        try:
            fn()
        except mi.Mi355Error as e:
            return e.status
        return 0

    INVALID, UNSUP = -4, -3
    buf = torch.empty(want + 512, dtype=torch.uint8, device="cuda")
    base = buf.data_ptr() + (-buf.data_ptr()) % 256
    assert status(lambda: ctx.weight_prepare(wt, base + 16, want)) == INVALID       # dst not 256-aligned
    assert status(lambda: ctx.weight_prepare(wt, base, want - 1)) == INVALID        # dst too small
    assert status(lambda: ctx.weight_prepare(pt, base, want)) == INVALID            # already prepared
    w3 = mi.from_torch(dev(np.concatenate([wq, wq]).view(np.uint8)), t, [K, N, 2])  # 3-D weight
    assert mi.weight_prepared_nbytes(w3) == 0
    assert status(lambda: ctx.weight_prepare(w3, base, want * 2)) == INVALID
    x3 = torch.zeros((2, M, K), device="cuda")
    d3 = torch.zeros((2, M, N), device="cuda")
    assert status(lambda: ctx.mul_mat(pt, mi.from_torch(x3, mi.F32, [K, M, 2]),
                                      mi.from_torch(d3, mi.F32, [N, M, 2]))) == UNSUP
    # a prepared tensor is not a ggml tensor for any other operand or op
    assert status(lambda: ctx.mul_mat(wt, pt, mi.from_torch(outs[0], mi.F32, [N, M]))) == INVALID
    assert status(lambda: ctx.quantize_rows(t, mi.ACT_X86, pt, base)) == INVALID
    qf = torch.zeros((64, 4), dtype=torch.float16, device="cuda")
    of = torch.zeros((4, 64), dtype=torch.float32, device="cuda")
    qt = mi.from_torch(qf, mi.F16, [64, 4, 1, 1])
    fake = mi.make_tensor(qf.data_ptr(), mi.F16, [64, 4, 1, 1])
    fake.layout = mi.LAYOUT_INT8
    assert status(lambda: ctx.flash_attn_ext(fake, qt, qt, mi.from_torch(of, mi.F32, [64, 1, 4, 1]), 0.125)) == INVALID


@pytest.mark.parametrize("route,tname", [("f16", "q8_0"), ("f16", "q4_1"), ("f16", "f16"), ("int8", "q8_0"),
                                         ("int8", "q4_1")])
@pytest.mark.parametrize("M,K", [(5184, 1024), (77, 96), (301, 4736)])
def test_flat_and_strided_activations_bit_identical(mi, ctx, orc, route, tname, M, K):
    """src1 rows at a 16-byte aligned pitch take the vector-load paths of the
    activation conversions (quantize_mmq_kernel's float4 loads,
    convert_f16_flat_kernel), rows at an odd pitch the element-wise ones; both
    are ggml's from_float, so the products must be equal bit for bit (F16
    weights have no int8 route)."""
    t = orc.NAME_TYPE[tname]
    N = 96
    print(f"flat vs strided src1 {route} {tname} M={M} K={K}", flush=True)
    w = orc.normal(N * K, seed=K + M, stream=1, std=0.02).reshape(N, K)
    x = orc.normal(M * K, seed=K + M, stream=2).reshape(M, K)
    wq = orc.quantize_weights(t, w) if t != orc.F16 else w.astype(np.float16).view(np.uint16)
    s0 = mi.from_torch(dev(wq.view(np.uint8)), t, [K, N])
    flat = dev(x)
    wide = torch.zeros((M, K + 1), dtype=torch.float32, device="cuda")
    wide[:, :K] = flat
    outs = []
    ctx.set_mmq_kernel(_kernel(mi, route))
    try:
        for src, nb1 in ((flat, 4 * K), (wide, 4 * (K + 1))):
            dst = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
            s1 = mi.from_torch(src, mi.F32, [K, M], nb=[4, nb1, nb1 * M, nb1 * M])
            ctx.mul_mat(s0, s1, mi.from_torch(dst, mi.F32, [N, M]))
            ctx.synchronize()
            outs.append(dst)
    finally:
        ctx.set_mmq_kernel(mi.MMQ_AUTO)
    assert torch.isfinite(outs[0]).all()
    assert torch.equal(outs[0], outs[1]), f"max diff {(outs[0] - outs[1]).abs().max().item():.3e}"
