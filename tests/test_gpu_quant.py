"""GPU activation quantize (mi355_quantize_rows) is bit-exact with the
oracle's ggml from_float: Q8_0 / Q8_1 in both the x86 (half-even) and _ref
(half-away) variants, and F16 (round to nearest even)."""
import json
import os

import numpy as np
import pytest
import torch

from gpu_helpers import dev

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def gpu_quantize(mi, ctx, t, variant, x, nb=None, ne=None):
    xd = dev(x)
    rows = int(np.prod(x.shape[:-1])) if ne is None else ne[1] * ne[2] * ne[3]
    k = x.shape[-1] if ne is None else ne[0]
    rs = mi.row_size(t, k)
    out = torch.zeros(rows * rs + 16, dtype=torch.uint8, device="cuda")
    src = mi.from_torch(xd, mi.F32, ne or [k, rows], nb)
    ctx.quantize_rows(t, variant, src, out.data_ptr())
    ctx.synchronize()
    return out[: rows * rs].cpu().numpy().reshape(rows, rs)


def special_rows(orc):
    rows = []
    with open(os.path.join(HERE, "golden", "quant_kat.json")) as f:
        kat = json.load(f)
    for c in kat["q8_act"]:
        rows.append(np.array(c["x"], dtype=np.float32))
    z = np.zeros(32, np.float32)
    spike = z.copy(); spike[7] = -3.7
    tiny = np.full(32, 1e-30, np.float32); tiny[0] = -2e-30
    huge = orc.normal(32, 9, 9) * np.float32(1e4)
    rows += [z, spike, tiny, huge]
    return np.concatenate(rows)


@pytest.mark.parametrize("t,variant", [("q8_0", 0), ("q8_0", 1), ("q8_1", 0), ("q8_1", 1), ("f16", 0)])
def test_quantize_bit_exact(mi, ctx, orc, t, variant):
    """Both from_float variants (x86, _ref) of Q8_0 / Q8_1; F16 has only one."""
    t = orc.NAME_TYPE[t]
    K = 1024
    x = orc.normal(96 * K, seed=1, stream=5).reshape(96, K) * np.float32(2.5)
    sp = special_rows(orc)
    x[0, : sp.size] = sp
    ref = orc.from_float(t, x, variant)
    out = gpu_quantize(mi, ctx, t, variant, x)
    bad = np.nonzero((out != ref).any(axis=1))[0]
    assert bad.size == 0, f"rows differ: {bad[:8]}"


def test_quantize_strided_source(mi, ctx, orc):
    """src as a transposed view (nb0 = 4*rows): same bytes as the contiguous copy."""
    K, R = 256, 40
    xt = orc.normal(K * R, seed=2, stream=1).reshape(K, R)  # memory [K][R]
    out = gpu_quantize(mi, ctx, orc.Q8_0, 0, xt, nb=[4 * R, 4, 4 * R * K, 4 * R * K], ne=[K, R, 1, 1])
    ref = orc.from_float(orc.Q8_0, np.ascontiguousarray(xt.T), 0)
    assert np.array_equal(out, ref)


def test_quantize_config_shape(mi, ctx, orc):
    """The fc1 activation [5184 x 1024] N(0,1), seed 0: all 5.64 MB of Q8_0 bytes."""
    x = orc.normal(5184 * 1024, seed=0, stream=2).reshape(5184, 1024)
    ref = orc.from_float(orc.Q8_0, x, 0)
    out = gpu_quantize(mi, ctx, orc.Q8_0, 0, x)
    assert np.array_equal(out, ref)
