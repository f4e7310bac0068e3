"""Pins the oracle's ggml_mul_mat restatement (src1 -> vec_dot_type, then
vec_dot per (row, col), ne2/ne3 broadcast) against numpy float64 computed
from an independent numpy decoder of the block bytes.

Tolerance: |oracle - ref| <= 1e-6 * absterm, where absterm is the sum of the
absolute elementwise terms sum_b |d_w d_a| sum_j |q_w q_a| (+|m_w s_a|) -- the
scale that bounds the rounding error of any fp32 summation order (outputs
near 0 make a per-element relative error meaningless).
"""
import ctypes as C

import numpy as np
import pytest


def ref_mul_mat(orc, t, wq, K, xq):
    """float64 ggml block formula from decoded blocks: [M, N]."""
    if t == orc.F16:
        w = wq.view(np.float16).astype(np.float64).reshape(-1, K)
        x = xq.view(np.float16).astype(np.float64).reshape(-1, K)
        return x @ w.T, np.abs(x) @ np.abs(w).T
    vt = orc.VEC_DOT_TYPE[t]
    wv, wd, wm = orc.decode_blocks(t, wq, K)
    xv, xd, xs = orc.decode_blocks(vt, xq, K)
    nb = K // 32
    # isum[m, n, b]
    xb = xv.reshape(-1, nb, 32).astype(np.int64)
    wb = wv.reshape(-1, nb, 32).astype(np.int64)
    isum = np.einsum("mbj,nbj->mnb", xb, wb).astype(np.float64)
    iabs = np.einsum("mbj,nbj->mnb", np.abs(xb), np.abs(wb)).astype(np.float64)
    dd = xd[:, None, :].astype(np.float64) * wd[None, :, :].astype(np.float64)
    terms, aterms = isum * dd, iabs * np.abs(dd)
    if t == orc.Q4_1:
        ms = xs[:, None, :].astype(np.float64) * wm[None, :, :].astype(np.float64)
        terms, aterms = terms + ms, aterms + np.abs(ms)
    # absterm: sum of |elementwise terms|, the scale of any summation order's rounding error
    return terms.sum(axis=2), aterms.sum(axis=2)


@pytest.mark.parametrize("tname", ["q8_0", "q4_0", "q4_1", "f16"])
@pytest.mark.parametrize("K", [32, 96, 1024])
def test_mul_mat_vs_block_formula(orc, tname, K):
    t = orc.NAME_TYPE[tname]
    N, M = 40, 24
    w = orc.normal(N * K, seed=0, stream=1, std=0.02).reshape(N, K)
    x = orc.normal(M * K, seed=0, stream=2).reshape(M, K)
    wq = orc.quantize_weights(t, w)
    for order in (orc.ORDER_X86, orc.ORDER_SEQ):
        out = orc.mul_mat(wq, t, K, N, x[None, None], order=order)[0, 0]
        xq = orc.from_float(orc.VEC_DOT_TYPE[t], x)
        ref, ab = ref_mul_mat(orc, t, wq, K, xq)
        assert np.all(np.abs(out - ref) <= 1e-6 * ab + 1e-30)
    ex, absterm = orc.mul_mat(wq, t, K, N, x[None, None], exact=True)
    assert np.all(np.abs(ex[0, 0] - ref) <= 1e-7 * ab + 1e-30)
    assert np.allclose(absterm[0, 0], ab, rtol=1e-6)


def test_mul_mat_broadcast_and_strides(orc):
    """ne12 = 2*ne02, ne13 = 3*ne03, and a non-contiguous src1 view."""
    t, K, N, M = orc.Q8_0, 64, 16, 8
    ne02, ne03, ne12, ne13 = 2, 1, 4, 3
    w = orc.normal(ne03 * ne02 * N * K, seed=1, stream=1, std=0.02).reshape(ne03 * ne02 * N, K)
    wq = orc.quantize_weights(t, w)
    x = orc.normal(ne13 * ne12 * M * K, seed=1, stream=2).reshape(ne13, ne12, M, K)
    out = orc.mul_mat(wq, t, K, N, x, dims=(ne02, ne03, ne12, ne13))
    wq4 = wq.reshape(ne03, ne02, N, -1)
    for i13 in range(ne13):
        for i12 in range(ne12):
            xq = orc.from_float(orc.Q8_0, x[i13, i12])
            ref, ab = ref_mul_mat(orc, t, wq4[i13 // (ne13 // ne03), i12 // (ne12 // ne02)], K, xq)
            assert np.all(np.abs(out[i13, i12] - ref) <= 1e-6 * ab)
    # src1 as a strided view: rows of a transposed [K, M] buffer (nb0 = 4*M)
    xt = np.ascontiguousarray(x[0, 0].T)  # [K, M]
    s0 = orc.tensor(wq, t, [K, N, 1, 1])
    s1 = orc.tensor(xt, orc.F32, [K, M, 1, 1], nb=[4 * M, 4, 4 * M * K, 4 * M * K])
    dst = np.zeros((M, N), dtype=np.float32)
    d = orc.tensor(dst, orc.F32, [N, M, 1, 1])
    assert orc.lib().orc_mul_mat(C.byref(s0), C.byref(s1), C.byref(d), 0, 0, 2) == 0
    assert np.array_equal(dst, out[0, 0, :, :] if ne02 == 1 else orc.mul_mat(wq[:N], t, K, N, x[:1, :1])[0, 0])


def test_mul_mat_rejects_bad_shapes(orc):
    wq = np.zeros((4, 34 * 2), dtype=np.uint8)
    x = np.zeros((3, 96), dtype=np.float32)
    dd = np.zeros((3, 4), dtype=np.float32)
    s0 = orc.tensor(wq, orc.Q8_0, [64, 4])
    s1 = orc.tensor(x, orc.F32, [96, 3])  # K mismatch
    d = orc.tensor(dd, orc.F32, [4, 3])
    assert orc.lib().orc_mul_mat(C.byref(s0), C.byref(s1), C.byref(d), 0, 0, 1) < 0
    s0 = orc.tensor(np.zeros(4 * 48, np.float32), orc.F32, [48, 4])
    s0.type = 2  # q4_0 with K % 32 != 0
    s1 = orc.tensor(np.zeros(3 * 48, np.float32), orc.F32, [48, 3])
    d = orc.tensor(np.zeros(12, np.float32), orc.F32, [4, 3])
    assert orc.lib().orc_mul_mat(C.byref(s0), C.byref(s1), C.byref(d), 0, 0, 1) < 0


def test_mul_mat_f16_src1(orc):
    """F16 x F16 (src1 already vec_dot_type) equals F16 x F32 after RNE conversion."""
    K, N, M = 64, 8, 5
    w = orc.normal(N * K, seed=2, stream=1, std=0.02).reshape(N, K)
    x = orc.normal(M * K, seed=2, stream=2).reshape(M, K)
    wq = orc.quantize_weights(orc.F16, w)
    a = orc.mul_mat(wq, orc.F16, K, N, x[None, None])
    xh = orc.fp16_bits(x)
    b = orc.mul_mat(wq, orc.F16, K, N, xh[None, None], src1_type=orc.F16)
    assert np.array_equal(a, b)
