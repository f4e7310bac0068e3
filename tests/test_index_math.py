"""The reciprocal division of the int8 kernel's fused epilogues (`div_rcp` in
sam3.cpp_amd/csrc/common.cuh): q = trunc(a * RN(1 / b)) in IEEE double, corrected by
one step either way, is a // b for a >= 0, b > 0, a + b < 2^31.  Python floats are IEEE
doubles with round-to-nearest, like the device's double multiply and division, so the
same steps run here; the cases include the quotient boundaries (a = k b - 1, k b, k b + 1)
where a truncation off by one shows, and divisors up to 2^30."""
import numpy as np


def div_rcp(a, b, rb):
    q = int(float(a) * rb)
    r = a - q * b
    if r < 0:
        q, r = q - 1, r + b
    elif r >= b:
        q, r = q + 1, r - b
    return q, r


def _check(a, b):
    assert a >= 0 and b > 0 and a + b < 2 ** 31
    assert div_rcp(a, b, 1.0 / float(b)) == divmod(a, b), (a, b)


def test_div_rcp_small_exhaustive():
    for b in range(1, 130):
        for a in range(0, 40 * b):
            _check(a, b)


def test_div_rcp_boundaries():
    rng = np.random.default_rng(7)
    divisors = [1, 2, 3, 7, 24, 576, 4096, 5184, 65535, 65536, 999983, 2 ** 20 + 1, 2 ** 29 - 3, 2 ** 30 - 1]
    divisors += [int(x) for x in rng.integers(1, 2 ** 30, 200)]
    for b in divisors:
        kmax = (2 ** 31 - 1 - b) // b
        for k in {0, 1, 2, kmax // 2, kmax - 1, kmax} | {int(x) for x in rng.integers(0, kmax + 1, 20)}:
            for a in (k * b - 1, k * b, k * b + 1, k * b + b // 2, k * b + b - 1):
                if 0 <= a and a + b < 2 ** 31:
                    _check(a, b)


def test_div_rcp_random():
    rng = np.random.default_rng(11)
    for _ in range(100000):
        b = int(rng.integers(1, 2 ** int(rng.integers(1, 31))))
        a = int(rng.integers(0, 2 ** 31 - b))
        _check(a, b)
