"""Shared helpers of the GPU parity tests: device buffers from numpy, calls
through the C-ABI, and the absolute-term scale the tolerances are stated
against."""
import numpy as np
import torch


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def run_mul_mat(mi, ctx, wq: np.ndarray, t: int, K: int, N: int, x: np.ndarray, dims=(1, 1, 1, 1),
                src1_type=None) -> np.ndarray:
    """ggml_mul_mat through mi355_mul_mat.  wq: stacked src0 rows (uint8 blocks / f16 bits);
    x: src1 [ne13, ne12, M, K] (float32 or float16); returns dst [ne13, ne12, M, N]."""
    ne02, ne03, ne12, ne13 = dims
    x = x.reshape(ne13, ne12, -1, K)
    M = x.shape[2]
    if src1_type is None:
        src1_type = mi.F16 if x.dtype == np.float16 else mi.F32
    w = dev(wq.view(np.uint8))
    xd = dev(x)
    dst = torch.full((ne13, ne12, M, N), float("nan"), dtype=torch.float32, device="cuda")
    s0 = mi.from_torch(w, t, [K, N, ne02, ne03])
    s1 = mi.from_torch(xd, src1_type, [K, M, ne12, ne13])
    d = mi.from_torch(dst, mi.F32, [N, M, ne12, ne13])
    ctx.mul_mat(s0, s1, d)
    ctx.synchronize()
    return dst.cpu().numpy()


def absterm(orc, t: int, wq: np.ndarray, K: int, xq: np.ndarray) -> np.ndarray:
    """sum_b |d_w d_a| sum_j |q_w q_a| (+ |m_w s_a|) per output [M, N], in float64:
    the scale bounding the rounding error of any fp32 summation order."""
    if t == orc.F16:
        w = np.abs(wq.view(np.float16).astype(np.float64).reshape(-1, K))
        x = np.abs(xq.view(np.float16).astype(np.float64).reshape(-1, K))
        return x @ w.T
    vt = orc.VEC_DOT_TYPE[t]
    nb = K // 32
    wv, wd, wm = orc.decode_blocks(t, wq, K)
    xv, xd, xs = orc.decode_blocks(vt, xq, K)
    wa = (np.abs(wv).reshape(-1, nb, 32) * np.abs(wd.astype(np.float64))[..., None]).reshape(-1, K)
    xa = (np.abs(xv).reshape(-1, nb, 32) * np.abs(xd.astype(np.float64))[..., None]).reshape(-1, K)
    a = xa @ wa.T
    if t == orc.Q4_1:
        a = a + np.abs(xs.astype(np.float64)) @ np.abs(wm.astype(np.float64)).T
    return a


def rel_err(out: np.ndarray, ref: np.ndarray, scale: np.ndarray) -> float:
    return float((np.abs(out.astype(np.float64) - ref) / np.maximum(scale, 1e-30)).max())
