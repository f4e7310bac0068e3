"""Pins the oracle's soft_max_ext and flash_attn_ext restatements.

Anchors: numpy float64 textbook softmax(scale QK^T)V; the long-double path
against numpy; key-permutation equivariance; ggml's own requirement that a
strided (permuted) V gives bit-identical output to a contiguous copy
(tests/test_v_cont_removal.cpp:156-160, tolerance 0.0).
"""
import numpy as np
import pytest


def np_attn(q, k, v, scale):
    # q [B, H, Nq, D], k [B, H, Nk, D], v [B, H, Nk, Dv] -> [B, Nq, H, Dv]
    s = np.einsum("bhqd,bhkd->bhqk", q.astype(np.float64), k.astype(np.float64)) * scale
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    o = np.einsum("bhqk,bhkd->bhqd", p, v.astype(np.float64))
    return o.transpose(0, 2, 1, 3)


def make_qkv(orc, B, H, Nq, Nk, D, dtype, seed=0):
    q = orc.normal(B * H * Nq * D, seed, 1).reshape(B, H, Nq, D)
    k = orc.normal(B * H * Nk * D, seed, 2).reshape(B, H, Nk, D)
    v = orc.normal(B * H * Nk * D, seed, 3).reshape(B, H, Nk, D)
    if dtype == "f16":
        q, k, v = (a.astype(np.float16) for a in (q, k, v))
    return q, k, v


def tens(orc, a):
    t = orc.F16 if a.dtype == np.float16 else orc.F32
    a = np.ascontiguousarray(a)
    B, H, N, D = a.shape
    return orc.tensor(a, t, [D, N, H, B])


def test_softmax(orc):
    x = orc.normal(6 * 333, 0, 9).reshape(2, 3, 333) * 4
    y = orc.soft_max_ext(x, 0.125)
    ref = np.exp(x.astype(np.float64) * 0.125 - (x.astype(np.float64) * 0.125).max(-1, keepdims=True))
    ref /= ref.sum(-1, keepdims=True)
    assert np.abs(y - ref).max() < 1e-6
    assert np.abs(y.sum(-1) - 1).max() < 1e-5


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_flash_attn_vs_textbook(orc, dtype):
    B, H, Nq, Nk, D = 2, 3, 20, 77, 64
    q, k, v = make_qkv(orc, B, H, Nq, Nk, D, dtype)
    scale = 1.0 / 8.0
    ref = np_attn(q, k, v, scale)
    ex = orc.flash_attn_ext(tens(orc, q), tens(orc, k), tens(orc, v), D, scale, exact=True)
    assert np.abs(ex - ref).max() < 1e-6
    out = orc.flash_attn_ext(tens(orc, q), tens(orc, k), tens(orc, v), D, scale)
    # f32 V accumulates in fp32; f16 V accumulates in fp16 (VKQ16) like ggml-cpu
    tol = 2e-5 if dtype == "f32" else 2e-2
    assert np.abs(out - ref).max() < tol


def test_flash_attn_key_permutation(orc):
    B, H, Nq, Nk, D = 1, 2, 9, 50, 64
    q, k, v = make_qkv(orc, B, H, Nq, Nk, D, "f32", seed=4)
    perm = np.random.default_rng(0).permutation(Nk)
    a = orc.flash_attn_ext(tens(orc, q), tens(orc, k), tens(orc, v), D, 0.125, exact=True)
    b = orc.flash_attn_ext(tens(orc, q), tens(orc, k[:, :, perm]), tens(orc, v[:, :, perm]), D, 0.125, exact=True)
    assert np.abs(a - b).max() < 1e-12
    # and the ggml loop order changes only rounding
    c = orc.flash_attn_ext(tens(orc, q), tens(orc, k[:, :, perm]), tens(orc, v[:, :, perm]), D, 0.125)
    assert np.abs(a - c).max() < 2e-5


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_flash_attn_strided_v_bit_identical(orc, dtype):
    """V as the permuted view of a [D, H, N, B] buffer vs a contiguous copy."""
    B, H, N, D = 2, 4, 30, 64
    q, k, v = make_qkv(orc, B, H, N, N, D, dtype, seed=7)
    base = np.ascontiguousarray(v.transpose(0, 2, 1, 3))  # [B, N, H, D]: ggml ne [D, H, N, B]
    ts = base.itemsize
    t = orc.F16 if dtype == "f16" else orc.F32
    v_view = orc.tensor(base, t, [D, N, H, B], nb=[ts, ts * D * H, ts * D, ts * D * H * N])
    a = orc.flash_attn_ext(tens(orc, q), tens(orc, k), v_view, D, 0.125)
    b = orc.flash_attn_ext(tens(orc, q), tens(orc, k), tens(orc, v), D, 0.125)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_flash_attn_gqa_broadcast(orc):
    """n_head_kv divides n_head: head h reads kv head h // (n_head / n_head_kv)."""
    B, H, Hkv, Nq, Nk, D = 1, 4, 2, 5, 11, 64
    q = orc.normal(B * H * Nq * D, 1, 1).reshape(B, H, Nq, D)
    k = orc.normal(B * Hkv * Nk * D, 1, 2).reshape(B, Hkv, Nk, D)
    v = orc.normal(B * Hkv * Nk * D, 1, 3).reshape(B, Hkv, Nk, D)
    out = orc.flash_attn_ext(tens(orc, q), tens(orc, k), tens(orc, v), D, 0.125, exact=True)
    ref = np_attn(q, np.repeat(k, 2, axis=1), np.repeat(v, 2, axis=1), 0.125)
    assert np.abs(out - ref).max() < 1e-6
