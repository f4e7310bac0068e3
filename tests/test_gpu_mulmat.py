"""GPU mul_mat parity through the C-ABI (mi355_mul_mat) against the oracle's
ggml-cpu restatement on identical seeded inputs.

Bars (from the path's contract):
  * integer block dots: bit-exact (mi355_mul_mat_block_dots vs numpy int64);
  * quantized paths:   |gpu - oracle| <= 1e-5 * absterm
  * F16:               |gpu - oracle| <= 2e-3 * absterm
absterm = sum_b |d_w d_a| sum_j |q_w q_a| (+|m_w s_a|), the scale that bounds
the fp32 rounding of any summation order (outputs near zero make a plain
per-element relative error meaningless).
"""
import numpy as np
import pytest
import torch

from gpu_helpers import absterm, dev, rel_err, run_mul_mat

pytestmark = pytest.mark.gpu
TOL = {"q8_0": 1e-5, "q4_0": 1e-5, "q4_1": 1e-5, "f16": 2e-3}


def check(mi, ctx, orc, tname, M, N, K, seed=0, dims=(1, 1, 1, 1), wstd=0.02, xscale=1.0, sample=None):
    t = orc.NAME_TYPE[tname]
    ne02, ne03, ne12, ne13 = dims
    w = orc.normal(ne03 * ne02 * N * K, seed=seed, stream=1, std=wstd).reshape(-1, K)
    x = orc.normal(ne13 * ne12 * M * K, seed=seed, stream=2).reshape(ne13, ne12, M, K) * np.float32(xscale)
    wq = orc.quantize_weights(t, w)
    out = run_mul_mat(mi, ctx, wq, t, K, N, x, dims)
    assert np.isfinite(out).all()
    vt = orc.VEC_DOT_TYPE[t]
    wq4 = wq.reshape(ne03, ne02, N, -1)
    worst = 0.0
    for i13 in range(ne13):
        for i12 in range(ne12):
            rows = np.arange(M) if sample is None else sample
            xs = x[i13, i12, rows]
            wb = wq4[i13 // (ne13 // ne03), i12 // (ne12 // ne02)]
            ref = orc.mul_mat(wb, t, K, N, xs[None, None])[0, 0]
            xq = orc.from_float(vt, xs)
            scale = absterm(orc, t, wb, K, xq)
            e = rel_err(out[i13, i12, rows], ref, scale)
            worst = max(worst, e)
    assert worst <= TOL[tname], f"{tname} M={M} N={N} K={K}: rel err {worst:.3e}"
    return worst


@pytest.mark.parametrize("tname", ["q8_0", "q4_0", "q4_1", "f16"])
@pytest.mark.parametrize("M,N,K", [(1, 1, 32), (77, 65, 96), (128, 128, 128), (200, 300, 1024), (33, 130, 4736)])
def test_mul_mat_small(mi, ctx, orc, tname, M, N, K):
    check(mi, ctx, orc, tname, M, N, K)


@pytest.mark.parametrize("tname", ["q8_0", "q4_0", "q4_1", "f16"])
def test_mul_mat_broadcast(mi, ctx, orc, tname):
    # src0 [K, N, 2, 1] broadcast over src1 [K, M, 4, 3]
    check(mi, ctx, orc, tname, 40, 72, 256, seed=3, dims=(2, 1, 4, 3))


@pytest.mark.parametrize("tname", ["q8_0", "q4_0", "q4_1"])
@pytest.mark.parametrize("K", [96, 1024])
def test_block_dots_bit_exact(mi, ctx, orc, tname, K):
    t = orc.NAME_TYPE[tname]
    M, N = 70, 45
    w = orc.normal(N * K, seed=4, stream=1, std=0.02).reshape(N, K)
    x = orc.normal(M * K, seed=4, stream=2).reshape(M, K)
    wq = orc.quantize_weights(t, w)
    nb = K // 32
    isums = torch.zeros(M * N * nb, dtype=torch.int32, device="cuda")
    s0 = mi.from_torch(dev(wq), t, [K, N])
    s1 = mi.from_torch(dev(x), mi.F32, [K, M])
    ctx.mul_mat_block_dots(s0, s1, isums.data_ptr())
    ctx.synchronize()
    got = isums.cpu().numpy().reshape(M, N, nb)
    wv, _, _ = orc.decode_blocks(t, wq, K)
    xv, _, _ = orc.decode_blocks(orc.VEC_DOT_TYPE[t], orc.from_float(orc.VEC_DOT_TYPE[t], x), K)
    ref = np.einsum("mbj,nbj->mnb", xv.reshape(M, nb, 32).astype(np.int64), wv.reshape(N, nb, 32).astype(np.int64))
    assert np.array_equal(got, ref)


def test_integer_exact_through_product_path(mi, ctx, orc):
    """Scales of exactly 1.0 on both sides make the fp32 result an exact
    integer: activations are integers in [-127,127] with |127| in every block
    (d_a = 1, id = 1), weights are Q8_0 blocks with d = 1.0.  The GPU output
    must equal sum_b isum_b bit for bit."""
    M, N, K = 96, 80, 1024
    rng = np.random.default_rng(11)
    x = rng.integers(-127, 128, size=(M, K)).astype(np.float32)
    x.reshape(M, K // 32, 32)[:, :, 5] = 127.0
    q = rng.integers(-127, 128, size=(N, K)).astype(np.int8)
    wq = np.zeros((N, K // 32, 34), dtype=np.uint8)
    wq[:, :, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    wq[:, :, 2:] = q.reshape(N, K // 32, 32).view(np.uint8)
    out = run_mul_mat(mi, ctx, wq.reshape(N, -1), orc.Q8_0, K, N, x[None, None])[0, 0]
    exact = x.astype(np.int64) @ q.astype(np.int64).T
    assert np.abs(exact).max() < 2**24
    assert np.array_equal(out, exact.astype(np.float32))


@pytest.mark.parametrize("M,N,K", [(300, 64, 588), (77, 40, 147), (5, 3, 3), (130, 200, 1004)])
def test_mul_mat_f16_ragged_k(mi, ctx, orc, M, N, K):
    """F16 weights whose K is not a multiple of 8 (the 14x14x3 patch-embed
    conv, K = 588; the 7x7x3 stem, K = 147): rows are only 2-byte aligned, are
    copied to a zero-padded pitch, and the F16 activation rows are padded
    with zeros to the same pitch; same bar as every F16 shape."""
    check(mi, ctx, orc, "f16", M, N, K, seed=7)


@pytest.mark.parametrize("K", [64, 147])
def test_f16_src1_direct(mi, ctx, orc, K):
    """F16 src1 (the explicit attention form multiplies f16 K by f16 Q); a K
    that is not a multiple of 8 takes the padded copy of src1."""
    N, M = 200, 150
    w = orc.normal(N * K, seed=5, stream=1).reshape(N, K).astype(np.float16)
    x = orc.normal(M * K, seed=5, stream=2).reshape(M, K).astype(np.float16)
    out = run_mul_mat(mi, ctx, w.view(np.uint16), orc.F16, K, N, x[None, None])[0, 0]
    ref = orc.mul_mat(w.view(np.uint16), orc.F16, K, N, x.view(np.uint16)[None, None], src1_type=orc.F16)[0, 0]
    scale = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    assert rel_err(out, ref, scale) <= 2e-3


@pytest.mark.parametrize("tname", ["q8_0", "q4_0", "q4_1", "f16"])
@pytest.mark.parametrize("name,N,K", [("qkv", 3072, 1024), ("proj", 1024, 1024), ("fc1", 4736, 1024),
                                      ("fc2", 1024, 4736)])
def test_mul_mat_vit_shapes(mi, ctx, orc, tname, name, N, K):
    """SAM3 ViT block linear set at M = 5184 tokens (72x72), weights
    N(0,0.02), activations N(0,1), seed 0; 192 sampled token rows compared
    against the oracle (all N columns)."""
    sample = np.random.default_rng(0).choice(5184, size=192, replace=False)
    sample.sort()
    sample[0], sample[-1] = 0, 5183
    check(mi, ctx, orc, tname, 5184, N, K, seed=0, sample=sample)


@pytest.mark.parametrize("tname", ["q8_0", "q4_0", "q4_1", "f16"])
@pytest.mark.parametrize("M,N,K", [(1024, 768, 3072), (4096, 384, 1536), (96, 80, 4736)])
def test_mul_mat_split_k(mi, ctx, orc, tname, M, N, K):
    """Few output tiles over a long K (Hiera-tiny stage-3 fc2, stage-2 fc2, a
    single tile): the K range is split over workgroups and the partial sums
    are added by a reduction; same bars as every other shape."""
    sample = np.random.default_rng(1).choice(M, size=min(M, 128), replace=False)
    sample.sort()
    sample[0], sample[-1] = 0, M - 1
    check(mi, ctx, orc, tname, M, N, K, seed=3, sample=sample)


@pytest.mark.parametrize("tname", ["q8_0", "q4_0", "q4_1", "f16"])
@pytest.mark.parametrize("M,N,K", [(65536, 288, 96), (5000, 100, 64), (4097, 33, 128), (8192, 384, 32),
                                   (16384, 192, 96)])
def test_mul_mat_skinny(mi, ctx, orc, tname, M, N, K):
    """K <= 128 at M >= 4096 (SAM2 Hiera-tiny stage 1: 65536 tokens, K = 96,
    qkv N = 288) with quantized weights runs on the skinny kernel:
    bit-identical to the tiled kernel (same instruction sequence per 32x32
    tile), and within the usual bar of the oracle on sampled rows (ragged M
    and N included).  F16 weights stay on the tiled kernel (both calls)."""
    t = orc.NAME_TYPE[tname]
    w = orc.normal(N * K, seed=9, stream=1, std=0.02).reshape(N, K)
    x = orc.normal(M * K, seed=9, stream=2).reshape(M, K)
    wq = orc.quantize_weights(t, w)
    got = run_mul_mat(mi, ctx, wq, t, K, N, x[None, None])[0, 0]
    ctx.set_skinny(False)
    try:
        tiled = run_mul_mat(mi, ctx, wq, t, K, N, x[None, None])[0, 0]
    finally:
        ctx.set_skinny(True)
    assert np.array_equal(got, tiled)
    rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(M).choice(M, 128, replace=False)]))
    ref = orc.mul_mat(wq, t, K, N, x[rows][None, None])[0, 0]
    scale = absterm(orc, t, wq, K, orc.from_float(orc.VEC_DOT_TYPE[t], x[rows]))
    assert rel_err(got[rows], ref, scale) <= TOL[tname]


def _sweep_shapes(tname, n=16, seed=2024):
    """Seeded random GEMM shapes: ragged M and N, odd block counts, K up to 1280,
    F16 with any K, and now and then a broadcast batch (src0 [K,N,2,1] over src1
    [K,M,2,3])."""
    rng = np.random.default_rng(seed + sum(map(ord, tname)))
    out = []
    for i in range(n):
        M = int(rng.integers(1, 700))
        N = int(rng.integers(1, 520))
        K = int(rng.integers(1, 1281)) if tname == "f16" else 32 * int(rng.integers(1, 41))
        dims = (2, 1, 2, 3) if i % 5 == 4 else (1, 1, 1, 1)
        out.append((M, N, K, dims, i))
    return out


@pytest.mark.parametrize("tname", ["q8_0", "q4_0", "q4_1", "f16"])
def test_mul_mat_random_shapes(mi, ctx, orc, tname):
    for M, N, K, dims, i in _sweep_shapes(tname):
        check(mi, ctx, orc, tname, M, N, K, seed=100 + i, dims=dims)


def test_q8_1_sum_midpoint_rounding(mi, ctx, orc):
    """Q4_1 weights take the Q8_1 operand, whose s = fp16(d * isum) rounds the
    fp32 product first (ggml's from_float).  For this block (values from the
    oracle's seeded normal stream) d * isum in fp32 is exactly an fp16 midpoint,
    so rounding the exact product once instead of twice picks the other
    neighbour; the GPU once did that (a fused multiply-to-fp16).  One block per
    row makes that one-ulp s error ~1e-4 of the bar's scale."""
    x = orc.normal(6 * 420 * 288, seed=114, stream=2).reshape(3, 2, 420, 288)[1, 0, 29, 64:96].astype(np.float32)
    amax = np.float32(np.abs(x).max())
    d = np.float32(amax / np.float32(127.0))
    q = np.rint((x * (np.float32(127.0) / amax)).astype(np.float32)).astype(np.int64)
    p = np.float32(d * np.float32(q.sum()))
    lo = np.float16(p)
    hi = np.nextafter(lo, np.float16(np.inf) if np.float64(lo) < np.float64(p) else np.float16(-np.inf))
    assert np.float64(p) == (np.float64(lo) + np.float64(hi)) / 2, "not a midpoint case any more"
    K, N = 32, 64
    w = orc.normal(N * K, seed=7, stream=1, std=0.02).reshape(N, K)
    wq = orc.quantize_weights(orc.Q4_1, w)
    xs = np.tile(x, (3, 1))
    out = run_mul_mat(mi, ctx, wq, orc.Q4_1, K, N, xs[None, None])[0, 0]
    ref = orc.mul_mat(wq, orc.Q4_1, K, N, xs[None, None])[0, 0]
    scale = absterm(orc, orc.Q4_1, wq, K, orc.from_float(orc.Q8_1, xs))
    assert rel_err(out, ref, scale) <= TOL["q4_1"]


def test_two_contexts_two_threads(mi, orc):
    """One context per host thread and stream (the library's threading
    contract): two threads, each with its own context on its own stream, run
    interleaved mul_mats of different types and shapes (the skinny and tiled
    kernels, split-K) 4 times each; every result is bit-identical to the same
    call made alone."""
    import threading
    cases = [("q4_0", 65536, 96, 96), ("q8_0", 700, 520, 1024), ("q4_1", 96, 80, 4736), ("f16", 300, 64, 588)]
    inputs = []
    for i, (tname, M, N, K) in enumerate(cases):
        t = orc.NAME_TYPE[tname]
        w = orc.quantize_weights(t, orc.normal(N * K, seed=50 + i, stream=1, std=0.02).reshape(N, K))
        x = orc.normal(M * K, seed=50 + i, stream=2).reshape(M, K)
        inputs.append((t, torch.from_numpy(w.view(np.uint8)).cuda(), torch.from_numpy(x).cuda(), M, N, K))

    def run(ctx, t, w, x, M, N, K):
        d = torch.empty((M, N), dtype=torch.float32, device="cuda")
        ctx.mul_mat(mi.from_torch(w, t, [K, N]), mi.from_torch(x, mi.F32, [K, M]), mi.from_torch(d, mi.F32, [N, M]))
        ctx.synchronize()
        return d

    solo = mi.Context(0)
    try:
        ref = [run(solo, *a).cpu() for a in inputs]
    finally:
        solo.close()
    results, errors = {}, []

    def worker(tid):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                ctx = mi.Context(0, s.cuda_stream)
                try:
                    for rep in range(4):
                        for i in range(tid, tid + len(inputs)):
                            j = i % len(inputs)
                            results[(tid, rep, j)] = run(ctx, *inputs[j]).cpu()
                finally:
                    ctx.close()
        except Exception as e:  # reported below
            errors.append(repr(e))

    th = [threading.Thread(target=worker, args=(k,)) for k in range(2)]
    for x in th:
        x.start()
    for x in th:
        x.join(timeout=120)
    assert not errors, errors
    assert len(results) == 2 * 4 * len(inputs)
    for (tid, rep, j), out in results.items():
        assert torch.equal(out, ref[j]), (tid, rep, cases[j])
