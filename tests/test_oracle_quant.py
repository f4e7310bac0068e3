"""Pins the CPU oracle's fp16 conversion, block quantizers and block dots.

Anchors: numpy.float16 (an independent IEEE binary16 implementation),
hand-derived known-answer blocks (tests/golden/quant_kat.json), and
invariants that a transcription mistake (wrong tie rule, wrong sign of the
Q4_0 scale, swapped nibbles, dropped Q4_1 offset) breaks.
"""
import json
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def kat():
    with open(os.path.join(HERE, "golden", "quant_kat.json")) as f:
        return json.load(f)


def h(s):
    return int(s, 16)


# ---------------------------------------------------------------- fp16
def test_fp16_to_fp32_all_values(orc):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    out = np.empty(65536, dtype=np.float32)
    orc.lib().orc_fp16_to_fp32_row(bits.ctypes.data, out.ctypes.data, 65536)
    finite = np.isfinite(ref)
    assert np.array_equal(out[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.array_equal(np.isnan(out), np.isnan(ref))


def test_fp32_to_fp16_matches_numpy(orc):
    # every fp16 value, every midpoint between neighbouring fp16 values (the ties),
    # points just off the midpoints, and random float32 over the whole range
    b = np.arange(0, 0x7c00, dtype=np.uint32).astype(np.uint16)
    v = b.view(np.float16).astype(np.float64)
    mids = (v[:-1] + v[1:]) / 2.0
    cands = [v, mids, np.nextafter(mids, 0), np.nextafter(mids, 1e9)]
    rng = np.random.default_rng(0)
    rnd = rng.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = np.concatenate([c.astype(np.float32) for c in cands] + [rnd])
    x = np.concatenate([x, -x])
    x = x[~np.isnan(x)]
    ref = x.astype(np.float16).view(np.uint16)
    out = orc.fp16_bits(x)
    bad = np.nonzero(out != ref)[0]
    assert bad.size == 0, [(float(x[i]), hex(out[i]), hex(ref[i])) for i in bad[:5]]


def test_fp16_kat(orc, kat):
    for fbits, hbits in kat["fp16"]:
        f = np.array([h(fbits)], dtype=np.uint32).view(np.float32)
        assert int(orc.fp16_bits(f)[0]) == h(hbits), (fbits, hbits)


# ---------------------------------------------------------------- activation quantizers
def _blk(raw, t):
    return raw.reshape(-1)


@pytest.mark.parametrize("variant,key", [(0, "x86"), (1, "ref")])
def test_q8_act_kat(orc, kat, variant, key):
    for case in kat["q8_act"]:
        x = np.array(case["x"], dtype=np.float32)[None, :]
        q0 = orc.from_float(orc.Q8_0, x, variant)[0]
        assert int(q0[0:2].view(np.uint16)[0]) == h(case["d"]), case["name"]
        assert q0[2:34].view(np.int8).tolist() == case["qs_" + key], case["name"]
        q1 = orc.from_float(orc.Q8_1, x, variant)[0]
        assert int(q1[0:2].view(np.uint16)[0]) == h(case["d"]), case["name"]
        assert int(q1[2:4].view(np.uint16)[0]) == h(case["s_" + key]), case["name"]
        assert q1[4:36].view(np.int8).tolist() == case["qs_" + key], case["name"]


def test_q8_weight_quantizer_is_ref_variant(orc, kat):
    # ggml_quantize_chunk -> quantize_row_q8_0_ref (examples/quantize.cpp:244-245)
    for case in kat["q8_act"]:
        x = np.array(case["x"], dtype=np.float32)[None, :]
        q = orc.quantize_weights(orc.Q8_0, x)[0]
        assert q[2:34].view(np.int8).tolist() == case["qs_ref"]


def test_q8_properties(orc):
    x = orc.normal(64 * 1024, seed=3, stream=7).reshape(64, 1024) * np.float32(3.0)
    for variant in (orc.ACT_X86, orc.ACT_REF):
        q = orc.from_float(orc.Q8_0, x, variant)
        vals, d, _ = orc.decode_blocks(orc.Q8_0, q, 1024)
        xb = x.reshape(64, 32, 32)
        vb = vals.reshape(64, 32, 32)
        # the amax element quantizes to +-127, all |q| <= 127
        amax_idx = np.abs(xb).argmax(axis=2)
        at = np.take_along_axis(vb, amax_idx[..., None], axis=2)[..., 0]
        assert np.all(np.abs(at) == 127)
        assert np.abs(vb).max() <= 127
        # d == fp16(amax/127)
        amax = np.abs(xb).max(axis=2)
        assert np.array_equal(d, (amax / np.float32(127)).astype(np.float16).astype(np.float32))
        # reconstruction within half a step of the fp32 scale (plus fp16 rounding of d)
        err = np.abs(vb * (amax / 127)[..., None] - xb)
        assert np.all(err <= (amax / 127)[..., None] * 0.5 * (1 + 1e-5))
        # signs agree
        assert np.all((np.sign(vb) == np.sign(xb)) | (vb == 0))
    # the two variants differ by at most one step, and only rarely
    a = orc.decode_blocks(orc.Q8_0, orc.from_float(orc.Q8_0, x, orc.ACT_X86), 1024)[0]
    b = orc.decode_blocks(orc.Q8_0, orc.from_float(orc.Q8_0, x, orc.ACT_REF), 1024)[0]
    assert np.abs(a - b).max() <= 1
    assert (a != b).mean() < 1e-3


def test_q8_1_sum(orc):
    x = orc.normal(16 * 256, seed=4, stream=1).reshape(16, 256)
    q = orc.from_float(orc.Q8_1, x)
    vals, d, s = orc.decode_blocks(orc.Q8_1, q, 256)
    # s uses the fp32 scale amax/127 (before its fp16 rounding): s = fp16(d32 * sum q)
    d32 = np.abs(x.reshape(16, 8, 32)).max(axis=2) / np.float32(127)
    expect = (d32 * vals.reshape(16, 8, 32).sum(axis=2).astype(np.float32)).astype(np.float16).astype(np.float32)
    assert np.array_equal(s, expect)
    # rounding d to fp16 first gives a different s on some blocks: the test can tell them apart
    wrong = (d * vals.reshape(16, 8, 32).sum(axis=2).astype(np.float32)).astype(np.float16).astype(np.float32)
    assert not np.array_equal(s, wrong)


# ---------------------------------------------------------------- weight quantizers
def test_q4_0_kat(orc, kat):
    for case in kat["q4_0"]:
        x = np.array(case["x"], dtype=np.float32)[None, :]
        q = orc.quantize_weights(orc.Q4_0, x)[0]
        assert int(q[0:2].view(np.uint16)[0]) == h(case["d"]), case["name"]
        assert q[2:18].tolist() == case["qs"], case["name"]
        deq = orc.dequantize(orc.Q4_0, q[None, :], 32)[0]
        assert deq.tolist() == case["deq"], case["name"]


def test_q4_1_kat(orc, kat):
    for case in kat["q4_1"]:
        x = np.array(case["x"], dtype=np.float32)[None, :]
        q = orc.quantize_weights(orc.Q4_1, x)[0]
        assert int(q[0:2].view(np.uint16)[0]) == h(case["d"]), case["name"]
        assert int(q[2:4].view(np.uint16)[0]) == h(case["m"]), case["name"]
        assert q[4:20].tolist() == case["qs"], case["name"]


def test_q4_first_extreme_wins(orc):
    """quantize_row_q4_0_ref / q4_1_ref scan with strict comparisons, so the
    FIRST of equal extremes is kept.  Hand-derived blocks:
    Q4_0 [2, -2, 0...]: max = +2, d = 2/-8 = -0.25 (fp16 0xb400), id = -4,
    q = (int)(x*id + 8.5): 2 -> 0, -2 -> (int)16.5 = 16 -> 15, 0 -> 8;
    [-2, 2, 0...]: max = -2, d = +0.25 (0x3400), id = 4: the same quants.
    Q4_1 [-0.0, 0.0, 1, 0...]: min = -0.0 (0.0 < -0.0 is false), m = 0x8000;
    d = 1/15 (fp16 0x2c44), id = 1/d = 14.999999, 1 -> (int)15.499999 = 15;
    [0.0, -0.0, 1, ...] keeps m = +0.0 (0x0000)."""
    z = np.zeros(32, np.float32)
    a = z.copy(); a[0], a[1] = 2.0, -2.0
    q = orc.quantize_weights(orc.Q4_0, a[None])[0]
    assert q[0:2].view(np.uint16)[0] == 0xB400
    assert q[2:18].tolist() == [0x80, 0x8F] + [0x88] * 14
    b = z.copy(); b[0], b[1] = -2.0, 2.0
    q = orc.quantize_weights(orc.Q4_0, b[None])[0]
    assert q[0:2].view(np.uint16)[0] == 0x3400
    assert q[2:18].tolist() == [0x80, 0x8F] + [0x88] * 14
    for first, m in ((-0.0, 0x8000), (0.0, 0x0000)):
        c = z.copy(); c[0], c[1], c[2] = first, -first, 1.0
        q = orc.quantize_weights(orc.Q4_1, c[None])[0]
        assert q[0:4].view(np.uint16).tolist() == [0x2C44, m]
        assert q[4:20].tolist() == [0, 0, 15] + [0] * 13


def test_q4_properties(orc):
    w = orc.normal(128 * 1024, seed=0, stream=11, std=0.02).reshape(128, 1024)
    wb = w.reshape(128, 32, 32)
    # Q4_0: nibbles in [0,15], d = -max/8 with max the signed extreme, |err| <= |d|/2 except the
    # clipped +7 side (q=16 -> 15) which can be off by up to |d|
    q = orc.quantize_weights(orc.Q4_0, w)
    vals, d, _ = orc.decode_blocks(orc.Q4_0, q, 1024)
    assert vals.min() >= -8 and vals.max() <= 7
    idx = np.abs(wb).argmax(axis=2)
    mx = np.take_along_axis(wb, idx[..., None], axis=2)[..., 0]
    assert np.array_equal(d, (mx / np.float32(-8)).astype(np.float16).astype(np.float32))
    deq = orc.dequantize(orc.Q4_0, q, 1024).reshape(128, 32, 32)
    err = np.abs(deq - wb)
    # reconstruction uses the fp16 d while quantization used fp32 d: slack |q-8|*|d|*2^-11 <= |d|/256
    ad = np.abs(d)[..., None]
    assert np.all(err <= ad * (1.0 + 2.0**-8))
    unclipped = vals.reshape(128, 32, 32) < 7
    assert np.all(err[unclipped] <= (ad * (0.5 + 2.0**-8)).repeat(32, axis=2)[unclipped])
    # the extreme element itself maps to q = -8 exactly (x*id + 8.5 = 0.5)
    at = np.take_along_axis(vals.reshape(128, 32, 32), idx[..., None], axis=2)[..., 0]
    assert np.all(at == -8)
    # Q4_1: m = fp16(min), d = fp16((max-min)/15), error <= d/2 (+ fp16 rounding of d and m)
    q = orc.quantize_weights(orc.Q4_1, w)
    vals, d, m = orc.decode_blocks(orc.Q4_1, q, 1024)
    assert vals.min() >= 0 and vals.max() <= 15
    assert np.array_equal(m, wb.min(axis=2).astype(np.float16).astype(np.float32))
    deq = orc.dequantize(orc.Q4_1, q, 1024).reshape(128, 32, 32)
    span = wb.max(axis=2) - wb.min(axis=2)
    assert np.all(np.abs(deq - wb) <= (span / 15)[..., None] * 0.5 + 1e-3 * span[..., None] + 1e-6)


def test_quantize_chunk_offsets(orc):
    # ggml_quantize_chunk(start, nrows) writes rows start/n_per_row .. +nrows in place
    w = orc.normal(8 * 64, seed=5, stream=0).reshape(8, 64)
    full = orc.quantize_weights(orc.Q8_0, w)
    out = np.zeros_like(full)
    L = orc.lib()
    for r0, nr in ((0, 3), (3, 2), (5, 3)):
        n = L.orc_quantize_chunk(orc.Q8_0, w.ctypes.data, out.ctypes.data, r0 * 64, nr, 64)
        assert n == nr * full.shape[1]
    assert np.array_equal(out, full)


# ---------------------------------------------------------------- block dots
def test_dot_kat(orc, kat):
    import ctypes as C
    L = orc.lib()
    for case in kat["dot"]:
        t = orc.NAME_TYPE[case["type"]]
        w = bytearray(np.array([h(case["w_d"])], dtype=np.uint16).tobytes())
        if t == orc.Q4_1:
            w += np.array([h(case["w_m"])], dtype=np.uint16).tobytes()
        w += bytes(np.array(case["w_qs"], dtype=np.int64).astype(np.int8 if t == orc.Q8_0 else np.uint8).tobytes())
        a = bytearray(np.array([h(case["a_d"])], dtype=np.uint16).tobytes())
        if t == orc.Q4_1:
            a += np.array([h(case["a_s"])], dtype=np.uint16).tobytes()
        a += bytes(np.array(case["a_qs"], dtype=np.int8).tobytes())
        wb = np.frombuffer(bytes(w), dtype=np.uint8).copy()
        ab = np.frombuffer(bytes(a), dtype=np.uint8).copy()
        isum = np.zeros(1, dtype=np.int32)
        assert L.orc_block_isums(t, 32, wb.ctypes.data, ab.ctypes.data, isum.ctypes.data) == 0
        assert int(isum[0]) == case["isum"]
        for order in (orc.ORDER_X86, orc.ORDER_SEQ):
            assert L.orc_vec_dot(t, 32, wb.ctypes.data, ab.ctypes.data, order) == case["dot"]


@pytest.mark.parametrize("t", ["q8_0", "q4_0", "q4_1"])
def test_block_isums_bruteforce(orc, t):
    t = orc.NAME_TYPE[t]
    K = 1024
    w = orc.normal(16 * K, seed=1, stream=2, std=0.02).reshape(16, K)
    x = orc.normal(4 * K, seed=1, stream=3).reshape(4, K)
    wq = orc.quantize_weights(t, w)
    xq = orc.from_float(orc.VEC_DOT_TYPE[t], x)
    wv, _, _ = orc.decode_blocks(t, wq, K)
    xv, _, _ = orc.decode_blocks(orc.VEC_DOT_TYPE[t], xq, K)
    out = np.zeros(K // 32, dtype=np.int32)
    for i in range(16):
        for j in range(4):
            orc.lib().orc_block_isums(t, K, wq[i].ctypes.data, xq[j].ctypes.data, out.ctypes.data)
            ref = (wv[i].reshape(-1, 32).astype(np.int64) * xv[j].reshape(-1, 32)).sum(axis=1)
            assert np.array_equal(out, ref)


@pytest.mark.parametrize("t", ["q8_0", "q4_0", "q4_1", "f16"])
def test_vec_dot_orders_and_isa(orc, t):
    """Both summation orders stay within 1e-6 of the absolute-term sum of the
    long-double block formula, and the AVX2 and AVX512-VNNI kernels (those the
    host has) are bit-identical to the scalar x86-order restatement."""
    t = orc.NAME_TYPE[t]
    K = 4736
    w = orc.normal(8 * K, seed=2, stream=1, std=0.02).reshape(8, K)
    x = orc.normal(8 * K, seed=2, stream=2).reshape(8, K)
    wq = orc.quantize_weights(t, w)
    xq = orc.from_float(orc.VEC_DOT_TYPE[t], x)
    L = orc.lib()
    L.orc_set_isa(-1)
    best = L.orc_isa_path()
    for i in range(8):
        for j in range(8):
            pw, px = wq[i].ctypes.data, xq[j].ctypes.data
            ex = L.orc_vec_dot_exact(t, K, pw, px)
            ab = L.orc_vec_dot_absterm(t, K, pw, px)
            L.orc_set_isa(0)
            s_x86 = L.orc_vec_dot(t, K, pw, px, orc.ORDER_X86)
            s_seq = L.orc_vec_dot(t, K, pw, px, orc.ORDER_SEQ)
            L.orc_set_isa(-1)
            assert abs(s_x86 - ex) <= 1e-6 * ab
            assert abs(s_seq - ex) <= 1e-6 * ab
            for path in range(1, best + 1):  # AVX2, then AVX512-VNNI where the host has them
                L.orc_set_isa(path)
                s_simd = L.orc_vec_dot(t, K, pw, px, orc.ORDER_X86)
                L.orc_set_isa(-1)
                assert np.float32(s_simd).view(np.uint32) == np.float32(s_x86).view(np.uint32), path


@pytest.mark.parametrize("t", ["q8_0", "q4_0", "q4_1"])
def test_vec_dot_simd_extremes(orc, t):
    """The SIMD dots on saturating operands: every quant at +-127 (Q8_0 both sides,
    the activation side for Q4) and the Q4 nibble extremes, random scales; each ISA
    path the host has returns the scalar x86-order bits."""
    t = orc.NAME_TYPE[t]
    K = 1024
    rng = np.random.default_rng(17)
    vt = orc.VEC_DOT_TYPE[t]
    L = orc.lib()
    L.orc_set_isa(-1)
    best = L.orc_isa_path()
    for trial in range(12):
        signs_w = rng.choice([-1.0, 1.0], size=K).astype(np.float32)
        signs_x = rng.choice([-1.0, 1.0], size=K).astype(np.float32)
        scale = np.float32(10.0 ** rng.uniform(-3, 2))
        w = (signs_w * scale).reshape(1, K)  # every block at +-amax: quants +-127 / nibble ends
        x = (signs_x * np.float32(rng.uniform(0.5, 4.0))).reshape(1, K)
        if trial % 3 == 1:
            x[0, ::7] = 0.0
        wq, xq = orc.quantize_weights(t, w), orc.from_float(vt, x)
        pw, px = wq[0].ctypes.data, xq[0].ctypes.data
        L.orc_set_isa(0)
        ref = L.orc_vec_dot(t, K, pw, px, orc.ORDER_X86)
        for path in range(1, best + 1):
            L.orc_set_isa(path)
            got = L.orc_vec_dot(t, K, pw, px, orc.ORDER_X86)
            assert np.float32(got).view(np.uint32) == np.float32(ref).view(np.uint32), (trial, path)
        L.orc_set_isa(-1)
