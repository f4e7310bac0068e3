"""GPU attention parity: FLASH_ATTN_EXT (sam3.cpp:3778, 4399) and the
explicit form mul_mat(K,Q) -> soft_max_ext -> mul_mat(V^T,KQ)
(sam3.cpp:8584-8589), through the C-ABI.

Tolerance (floating point, fp16 MFMA inputs, fp32 accumulation): with W the
exact attention of |V| (sum_j p_j |v_j|, per output element),
  |gpu - exact| <= 2e-3 * W + 1e-6
where exact is the long-double attention of the same fp16 inputs.  Against
the oracle's ggml-cpu restatement (which accumulates F16 V in fp16, VKQ16)
the bound adds that oracle's own distance from exact:
  |gpu - cpu| <= 2e-3 * W + |cpu - exact| + 1e-6.
F32 q/k/v enter the MFMAs rounded to fp16; against the exact attention of
the unrounded F32 inputs the bound is 6e-3 * W.
"""
import numpy as np
import pytest
import torch

from gpu_helpers import dev

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _f16(a):
    return np.ascontiguousarray(a.astype(np.float16))


def _inputs(orc, D, nq, nkv, nh, nhk, B, seed=0):
    q = orc.normal(B * nh * nq * D, seed, 40).reshape(B, nh, nq, D)
    k = orc.normal(B * nhk * nkv * D, seed, 41).reshape(B, nhk, nkv, D)
    v = orc.normal(B * nhk * nkv * D, seed, 42).reshape(B, nhk, nkv, D)
    return q, k, v


def _gpu_fa(mi, ctx, q, k, v, scale, qt, kvt, v_nb=None, v_ne=None, k_nb=None):
    """q/k/v numpy in [B, heads, n, D] order (or v given by raw buffer + ne/nb;
    with k_nb, k's rows are the first D elements of its last axis)."""
    B, nh, nq, D = q.shape
    qd, kd, vd = dev(q), dev(k), dev(v)
    nkv, nhk = k.shape[2], k.shape[1]
    dst = torch.full((B, nq, nh, D), float("nan"), dtype=torch.float32, device="cuda")
    tq = mi.from_torch(qd, qt, [D, nq, nh, B])
    tk = mi.from_torch(kd, kvt, [D, nkv, nhk, B], k_nb)
    tv = mi.from_torch(vd, kvt, v_ne or [D, nkv, nhk, B], v_nb)
    td = mi.from_torch(dst, mi.F32, [D, nh, nq, B])
    ctx.flash_attn_ext(tq, tk, tv, td, scale)
    ctx.synchronize()
    return dst.cpu().numpy()


def _oracle(orc, q, k, v, scale, t, exact):
    B, nh, nq, D = q.shape
    nkv, nhk = k.shape[2], k.shape[1]
    Q = orc.tensor(q, t, [D, nq, nh, B])
    K = orc.tensor(k, t, [D, nkv, nhk, B])
    V = orc.tensor(v, t, [D, nkv, nhk, B])
    return orc.flash_attn_ext(Q, K, V, D, scale, exact=exact)


def _bound_w(orc, q, k, v, scale):
    """exact attention of |V| with the same q, k: the per-element error scale."""
    return _oracle(orc, q, k, np.abs(v.astype(np.float32)), scale, orc.F32, True) if v.dtype == np.float32 else \
        _oracle(orc, q, k, np.abs(v), scale, orc.F16, True)


def _check(orc, got, q, k, v, scale, t):
    exact = _oracle(orc, q, k, v, scale, t, True)
    W = _bound_w(orc, q, k, v, scale)
    err = np.abs(got.astype(np.float64) - exact)
    assert np.isfinite(got).all()
    assert (err <= TOL * W + 1e-6).all(), f"max err/W {(err / np.maximum(W, 1e-30)).max():.3e}"
    cpu = _oracle(orc, q, k, v, scale, t, False)
    cerr = np.abs(cpu.astype(np.float64) - exact)
    assert (np.abs(got.astype(np.float64) - cpu) <= TOL * W + cerr + 1e-6).all()
    return float((err / np.maximum(W, 1e-30)).max())


@pytest.mark.parametrize("D,nq,nkv,nh,nhk,B", [
    (64, 1, 1, 1, 1, 1),
    (64, 37, 77, 2, 2, 1),
    (64, 128, 64, 1, 1, 1),
    (96, 100, 130, 4, 2, 2),      # grouped kv heads
    (128, 129, 65, 1, 1, 1),
    (64, 576, 576, 16, 16, 1),    # one SAM3 window, all heads
    (96, 196, 196, 4, 4, 3),      # Hiera 14x14 windows
    (96, 1024, 1024, 4, 4, 1),    # few query tiles: keys split over workgroups, then combined
    (64, 300, 2000, 2, 1, 1),     # uneven key ranges, grouped kv heads
    # at most 64 keys and 64 queries: one- and two-wavefront workgroups, one K/V buffer
    (96, 1, 1, 1, 1, 1),
    (96, 16, 16, 2, 2, 64),       # Hiera-tiny stage 1 (4x4 windows)
    (96, 4, 16, 4, 4, 64),        # the pooled stage-1 -> 2 block (4 queries per window)
    (96, 64, 64, 1, 1, 32),       # stage 0 (8x8 windows)
    (96, 49, 49, 8, 8, 25),       # stage 3 (7x7 windows)
    (96, 33, 64, 2, 1, 3),        # two wavefronts, grouped kv heads
])
def test_flash_attn_f16(mi, ctx, orc, D, nq, nkv, nh, nhk, B):
    q, k, v = (_f16(a) for a in _inputs(orc, D, nq, nkv, nh, nhk, B))
    scale = 1.0 / np.sqrt(D)
    got = _gpu_fa(mi, ctx, q, k, v, scale, mi.F16, mi.F16)
    _check(orc, got, q, k, v, scale, orc.F16)


def test_flash_attn_global_rows(mi, ctx, orc):
    """5184 keys, 16 heads (SAM3 global block); every query on the GPU, a
    sample of 40 queries per head against the oracle (rows are independent)."""
    D, n, nh = 64, 5184, 16
    q, k, v = (_f16(a) for a in _inputs(orc, D, n, n, nh, nh, 1, seed=3))
    scale = 0.125
    got = _gpu_fa(mi, ctx, q, k, v, scale, mi.F16, mi.F16)
    rows = np.linspace(0, n - 1, 40).astype(int)
    qs = np.ascontiguousarray(q[:, :, rows, :])
    # dst [B, nq, nh, D] -> rows of the sample
    _check(orc, np.ascontiguousarray(got[:, rows]), qs, k, v, scale, orc.F16)


def test_flash_attn_f32_vit_layout(mi, ctx, orc):
    """F32 Q, K contiguous and V the strided permute view of the qkv buffer
    (sam3.cpp:3762-3767: [HD, N, NH, B] with nb = [4, E*4, HD*4, E*N*4]).
    Strided V gives bit-identical output to a contiguous copy (the reference's
    tests/test_v_cont_removal.cpp property)."""
    HD, NH, N, B = 64, 4, 150, 2
    E = HD * NH
    q, k, _ = _inputs(orc, HD, N, N, NH, NH, B, seed=5)
    cur = orc.normal(B * N * E, 5, 43).reshape(B, N, E)  # V rows of the fused qkv output
    v_cont = np.ascontiguousarray(cur.reshape(B, N, NH, HD).transpose(0, 2, 1, 3))
    scale = 1.0 / np.sqrt(HD)
    got_strided = _gpu_fa(mi, ctx, q, k, cur, scale, mi.F32, mi.F32,
                          v_nb=[4, E * 4, HD * 4, E * N * 4], v_ne=[HD, N, NH, B])
    got_cont = _gpu_fa(mi, ctx, q, k, v_cont, scale, mi.F32, mi.F32)
    assert np.array_equal(got_strided, got_cont)
    # against the attention of the fp16-rounded inputs (what enters the MFMAs) ...
    qh, kh, vh = _f16(q), _f16(k), _f16(v_cont)
    _check(orc, got_cont, qh, kh, vh, scale, orc.F16)
    # ... and of the unrounded F32 inputs
    exact32 = _oracle(orc, q, k, v_cont, scale, orc.F32, True)
    W = _bound_w(orc, q, k, v_cont, scale)
    assert (np.abs(got_cont - exact32) <= 6e-3 * W + 1e-6).all()


def test_flash_attn_mixed_types_and_scale(mi, ctx, orc):
    """F32 Q with F16 K/V (ggml converts Q to K's type), negative and zero scale."""
    D, nq, nkv, nh = 64, 70, 90, 2
    q, k, v = _inputs(orc, D, nq, nkv, nh, nh, 1, seed=7)
    kh, vh = _f16(k), _f16(v)
    for scale in (-0.2, 0.0):
        got = _gpu_fa(mi, ctx, q, kh, vh, scale, mi.F32, mi.F16)
        _check(orc, got, _f16(q), kh, vh, scale, orc.F16)


@pytest.mark.parametrize("D", [64, 96, 128])
def test_flash_attn_k_row_strides(mi, ctx, orc, D):
    """F16 K rows inside wider rows (padding filled with NaN, never read): a row
    stride of 3D halves keeps 16-byte rows (K staged by LDS DMA), D + 2 does not
    (K staged through registers).  Both give output bit-identical to contiguous K."""
    nq, nkv, nh = 150, 200, 2
    q, k, v = (_f16(a) for a in _inputs(orc, D, nq, nkv, nh, nh, 1, seed=11))
    scale = 1.0 / np.sqrt(D)
    ref = _gpu_fa(mi, ctx, q, k, v, scale, mi.F16, mi.F16)
    _check(orc, ref, q, k, v, scale, orc.F16)
    for W in (3 * D, D + 2):
        kbuf = np.full((1, nh, nkv, W), np.nan, np.float16)
        kbuf[..., :D] = k
        got = _gpu_fa(mi, ctx, q, kbuf, v, scale, mi.F16, mi.F16, k_nb=[2, 2 * W, 2 * W * nkv, 2 * W * nkv * nh])
        assert np.array_equal(got, ref), f"row stride {W}"


@pytest.mark.parametrize("D", [64, 96, 128])
def test_flash_attn_k_row_strides_steady_state(mi, ctx, orc, D):
    """The same strided K through the staging loop's steady state: 2048 queries
    x 16 heads fill 256 workgroups, so the keys are not split over workgroups
    and each workgroup walks all 9 tiles of 576 keys (the next-but-one tile's
    load in flight behind the current one).  A row stride of 3D halves takes
    the K DMA staging, D + 2 the register staging; both must equal contiguous
    K bit for bit, and contiguous K must meet the oracle on sampled queries."""
    nq, nkv, nh = 2048, 576, 16
    q, k, v = (_f16(a) for a in _inputs(orc, D, nq, nkv, nh, nh, 1, seed=13))
    scale = 1.0 / np.sqrt(D)
    ref = _gpu_fa(mi, ctx, q, k, v, scale, mi.F16, mi.F16)
    rows = np.arange(0, nq, 97)
    _check(orc, np.ascontiguousarray(ref[:, rows]), np.ascontiguousarray(q[:, :, rows]), k, v, scale, orc.F16)
    for W in (3 * D, D + 2):
        kbuf = np.full((1, nh, nkv, W), np.nan, np.float16)
        kbuf[..., :D] = k
        got = _gpu_fa(mi, ctx, q, kbuf, v, scale, mi.F16, mi.F16, k_nb=[2, 2 * W, 2 * W * nkv, 2 * W * nkv * nh])
        assert np.array_equal(got, ref), f"row stride {W}"


def test_flash_attn_rejects(mi, ctx, orc):
    D, nq, nkv = 64, 8, 8
    q, k, v = (_f16(a) for a in _inputs(orc, D, nq, nkv, 1, 1, 1))
    qd, kd, vd = dev(q), dev(k), dev(v)
    dst = torch.empty((1, nq, 1, D), dtype=torch.float32, device="cuda")
    tq = mi.from_torch(qd, mi.F16, [D, nq, 1, 1])
    tk = mi.from_torch(kd, mi.F16, [D, nkv, 1, 1])
    tv = mi.from_torch(vd, mi.F16, [D, nkv, 1, 1])
    td = mi.from_torch(dst, mi.F32, [D, 1, nq, 1])
    import ctypes as C
    L = mi.lib()
    # mask -> UNSUPPORTED; softcap -> UNSUPPORTED; mismatched dst -> INVALID_ARG
    assert L.mi355_flash_attn_ext(ctx.h, C.byref(tq), C.byref(tk), C.byref(tv), C.byref(tq), 0.1, 0.0, 0.0,
                                  C.byref(td)) == -3
    assert L.mi355_flash_attn_ext(ctx.h, C.byref(tq), C.byref(tk), C.byref(tv), None, 0.1, 0.0, 30.0,
                                  C.byref(td)) == -3
    bad = mi.from_torch(dst, mi.F32, [D, nq, 1, 1])
    assert L.mi355_flash_attn_ext(ctx.h, C.byref(tq), C.byref(tk), C.byref(tv), None, 0.1, 0.0, 0.0,
                                  C.byref(bad)) == -4


@pytest.mark.parametrize("n,nh,nq_check", [(576, 16, 576), (5184, 16, 48)])
def test_explicit_attention_gemms(mi, ctx, orc, n, nh, nq_check):
    """KQ = mul_mat(K, Q) [n, n, nh], soft_max_ext(KQ, scale), KQV =
    mul_mat(cont(V^T), KQ) [D, n, nh] -- the batched QK^T / PV GEMMs with
    F16 K and V^T, F16 Q (the KQ probabilities are converted to F16 by the
    second mul_mat, as ggml-cpu's vec_dot_type for F16 src0)."""
    D = 64
    q, k, v = (_f16(a) for a in _inputs(orc, D, n, n, nh, nh, 1, seed=9))
    scale = 0.125
    qd, kd = dev(q[0]), dev(k[0])
    vt = dev(np.ascontiguousarray(v[0].transpose(0, 2, 1)))  # [nh, D, n]: cont(V^T)
    kq = torch.empty((nh, n, n), dtype=torch.float32, device="cuda")
    ctx.mul_mat(mi.from_torch(kd, mi.F16, [D, n, nh, 1]), mi.from_torch(qd, mi.F16, [D, n, nh, 1]),
                mi.from_torch(kq, mi.F32, [n, n, nh, 1]))
    ctx.soft_max_ext(mi.from_torch(kq, mi.F32, [n, n, nh, 1]), mi.from_torch(kq, mi.F32, [n, n, nh, 1]), scale)
    out = torch.empty((nh, n, D), dtype=torch.float32, device="cuda")
    ctx.mul_mat(mi.from_torch(vt, mi.F16, [n, D, nh, 1]), mi.from_torch(kq, mi.F32, [n, n, nh, 1]),
                mi.from_torch(out, mi.F32, [D, n, nh, 1]))
    ctx.synchronize()
    probs = kq.cpu().numpy()
    assert np.abs(probs.sum(-1) - 1).max() <= 1e-4
    rows = np.linspace(0, n - 1, nq_check).astype(int)
    got = out.cpu().numpy()[:, rows, :]                       # [nh, rows, D]
    qs = np.ascontiguousarray(q[:, :, rows, :])
    exact = _oracle(orc, qs, k, v, scale, orc.F16, True)[0]    # [rows, nh, D]
    W = _bound_w(orc, qs, k, v, scale)[0]
    err = np.abs(got.transpose(1, 0, 2).astype(np.float64) - exact)
    assert (err <= TOL * W + 1e-6).all(), f"max err/W {(err / np.maximum(W, 1e-30)).max():.3e}"


def test_flash_attn_random_shapes(mi, ctx, orc):
    """Seeded random shapes against the same bars: query and key counts ragged
    against the 128-query and 64-key tiles (some few enough that the keys are
    split over workgroups and combined), kv-head broadcast, D in {64, 96, 128},
    batches, and random scales."""
    rng = np.random.default_rng(4242)
    for i in range(14):
        D = int(rng.choice([64, 96, 128]))
        nq = int(rng.integers(1, 400))
        nkv = int(rng.integers(1, 900))
        nhk = int(rng.integers(1, 4))
        nh = nhk * int(rng.integers(1, 3))
        B = int(rng.integers(1, 3))
        scale = float(rng.uniform(0.05, 0.3))
        q, k, v = (_f16(a) for a in _inputs(orc, D, nq, nkv, nh, nhk, B, seed=200 + i))
        got = _gpu_fa(mi, ctx, q, k, v, scale, mi.F16, mi.F16)
        _check(orc, got, q, k, v, scale, orc.F16)
