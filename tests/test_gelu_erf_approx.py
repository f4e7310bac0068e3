"""The erf of the device GELU (`erf_gelu` in sam3.cpp_amd/csrc/common.cuh), restated in
float32 from the coefficients parsed out of that source: fmaf is emulated exactly (the
double product of two floats is exact, then one rounding to float32) and exp2 is taken
correctly rounded and one ulp off either way, the hardware's stated accuracy.  Against
scipy's erf it must stay within 9e-8 absolute on a sample of every 61st float32 in
[0, 4.5] and on every float32 around the piece boundary (1) and the clamp (4); past 4.5
the clamp gives 1 and erf(4.5) is within 2e-10 of 1, and erf is odd (copysign)."""
import os
import re

import numpy as np
from scipy.special import erf

SRC = os.path.join(os.path.dirname(__file__), "..", "sam3.cpp_amd", "csrc", "common.cuh")
f32 = np.float32


def _coefficients():
    src = open(SRC).read()
    body = src[src.index("float erf_gelu(float z)"):]
    body = body[:body.index("\n}\n")]
    lit = r"(-?[0-9.]+(?:e-?[0-9]+)?)f"
    p = [float(re.search(r"float p = " + lit, body).group(1))]
    p += [float(v) for v in re.findall(r"p = __builtin_fmaf\(p, t, " + lit + r"\)", body)]
    s = [float(re.search(r"float s = " + lit, body).group(1))]
    s += [float(v) for v in re.findall(r"s = __builtin_fmaf\(s, x, " + lit + r"\)", body)]
    c0 = float(re.search(r"__builtin_fmaf\(a, " + lit + r", a \* p\)", body).group(1))
    xc = float(re.search(r"const float x = a - " + lit, body).group(1))
    l2e = float(re.search(r"__builtin_fmaf\(t, " + lit + r", s\)", body).group(1))
    clamp = float(re.search(r"fminf\(fabsf\(z\), " + lit + r"\)", body).group(1))
    split = float(re.search(r"a < " + lit + r" \? ea : eb", body).group(1))
    assert len(p) == 7 and len(s) == 7
    return [f32(v) for v in p], [f32(v) for v in s], f32(c0), f32(xc), f32(l2e), f32(clamp), f32(split)


def _fma(a, b, c):
    return (np.asarray(a, np.float64) * np.asarray(b, np.float64) + np.asarray(c, np.float64)).astype(f32)


def erf_gelu(z, exp2_ulps=0):
    p, s, c0, xc, l2e, clamp, split = _coefficients()
    a = np.minimum(np.abs(z), clamp).astype(f32)
    t = (a * a).astype(f32)
    pp = np.full_like(t, p[0])
    for c in p[1:]:
        pp = _fma(pp, t, c)
    ea = _fma(a, c0, (a * pp).astype(f32))
    x = (a - xc).astype(f32)
    ss = np.full_like(x, s[0])
    for c in s[1:]:
        ss = _fma(ss, x, c)
    q = _fma(t, l2e, ss)
    e = np.exp2(-q.astype(np.float64)).astype(f32)
    for _ in range(abs(exp2_ulps)):
        e = np.nextafter(e, f32(np.inf) if exp2_ulps > 0 else f32(0)).astype(f32)
    eb = (f32(1.0) - e).astype(f32)
    return np.copysign(np.where(a < split, ea, eb), z).astype(f32)


def _inputs():
    lo, hi = int(f32(0).view(np.uint32)), int(f32(4.5).view(np.uint32))
    parts = [np.arange(lo, hi, 61, dtype=np.uint32)]
    for c in (1.0, 4.0):
        m = int(f32(c).view(np.uint32))
        parts.append(np.arange(m - 200000, m + 200000, dtype=np.uint32))
    return np.concatenate(parts).view(f32)


def test_erf_gelu_error_bound():
    z = _inputs()
    ref = erf(z.astype(np.float64))
    for ulps in (0, 1, -1):
        err = np.abs(erf_gelu(z, ulps).astype(np.float64) - ref)
        assert err.max() < 9e-8, (ulps, float(err.max()), float(z[np.argmax(err)]))


def test_erf_gelu_special_values():
    z = np.array([0.0, -0.0, 4.0, -4.0, 4.5, 1e30, -np.inf, np.inf, 1e-30, -1e-30], dtype=f32)
    got = erf_gelu(z)
    assert np.array_equal(np.signbit(got[:2]), [False, True]) and got[0] == 0.0
    assert np.array_equal(got[2:8], np.array([1, -1, 1, 1, -1, 1], dtype=f32))
    assert np.abs(got[8:] - erf(z[8:].astype(np.float64))).max() < 1e-37
