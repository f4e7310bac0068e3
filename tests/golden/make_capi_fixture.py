"""Writes tests/golden/capi_fixture.bin, the inputs and oracle results that
tests/native/capi_check.cpp (a C++ caller of the C-ABI with no torch and no
Python) uploads, runs and checks:

- mul_mat: Q8_0 weights [N=64 rows, K=128] quantized from f32 N(0, 0.02) by
  the oracle's quantize_row_q8_0_ref (ggml_quantize_chunk), activations f32
  N(0, 1) [M=32][K]; the oracle's ggml-cpu MUL_MAT result [M][N] and the
  absolute-term scale sum_b |d_w d_a| sum_j |q_w q_a| (float32) the 1e-5
  bar is stated against.
- flash_attn_ext: F16 q, k, v [B=1][n_head=2][n=40][D=64] from N(0, 1), scale
  1/8; exact attention of the fp16 operands [1][n][n_head][D] and the
  attention of |V| (the 2e-3 bar's scale).

Format: magic "MI355FX1", uint32 record count, then per record: a 32-byte
zero-padded name, uint32 element type (0 f32, 1 f16, 2 u8), uint32 zero,
uint64 byte count, the bytes, zero padding to a multiple of 8.
Run: python tests/golden/make_capi_fixture.py
"""
import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, os.path.dirname(HERE))

from oracle import oracle as orc  # noqa: E402
from gpu_helpers import absterm  # noqa: E402


def records():
    M, N, K = 32, 64, 128
    w = orc.normal(N * K, 400, 1, std=0.02).reshape(N, K)
    wq = orc.quantize_weights(orc.Q8_0, w)
    x = orc.normal(M * K, 400, 2).reshape(M, K)
    dst = orc.mul_mat(wq, orc.Q8_0, K, N, x[None, None])[0, 0]
    xq = orc.from_float(orc.Q8_0, x)
    at = absterm(orc, orc.Q8_0, wq, K, xq).astype(np.float32)
    D, n, nh = 64, 40, 2
    q, k, v = (orc.normal(nh * n * D, 401, s).reshape(1, nh, n, D).astype(np.float16) for s in (1, 2, 3))
    T = lambda a: orc.tensor(np.ascontiguousarray(a), orc.F16, [D, n, nh, 1])
    o = orc.flash_attn_ext(T(q), T(k), T(v), D, 0.125, exact=True)
    wabs = orc.flash_attn_ext(T(q), T(k), T(np.abs(v)), D, 0.125, exact=True)
    dims = np.array([M, N, K, D, n, nh], dtype=np.int32)
    return [("dims", 2, dims.view(np.uint8)), ("mm.w_q8_0", 2, wq), ("mm.x", 0, x), ("mm.dst", 0, dst),
            ("mm.absterm", 0, at), ("fa.q", 1, q), ("fa.k", 1, k), ("fa.v", 1, v), ("fa.out", 0, o),
            ("fa.wabs", 0, wabs)]


def main():
    out = os.path.join(HERE, "capi_fixture.bin")
    recs = records()
    with open(out, "wb") as f:
        f.write(b"MI355FX1" + struct.pack("<I", len(recs)))
        for name, et, arr in recs:
            b = np.ascontiguousarray(arr).tobytes()
            f.write(name.encode().ljust(32, b"\0") + struct.pack("<IIQ", et, 0, len(b)) + b)
            f.write(b"\0" * (-len(b) % 8))
    print(out, os.path.getsize(out))


if __name__ == "__main__":
    main()
