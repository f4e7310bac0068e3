"""ctypes binding of the CPU oracle (libggml_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py.  The product library never uses it.

The oracle restates ggml's CPU arithmetic for sam3.cpp's quantized mul_mat
path (sam3.cpp:3742-3799 emit the MUL_MAT nodes; ggml executes them).  This
module adds numpy conveniences: block encoders/decoders, synthetic inputs,
and orc_tensor views over numpy arrays.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libggml_oracle.so")

F32, F16, Q4_0, Q4_1, Q8_0, Q8_1 = 0, 1, 2, 3, 8, 9
ACT_X86, ACT_REF = 0, 1
ORDER_X86, ORDER_SEQ = 0, 1
QK = 32
TYPE_SIZE = {F32: 4, F16: 2, Q4_0: 18, Q4_1: 20, Q8_0: 34, Q8_1: 36}
BLCK = {F32: 1, F16: 1, Q4_0: 32, Q4_1: 32, Q8_0: 32, Q8_1: 32}
VEC_DOT_TYPE = {F32: F32, F16: F16, Q4_0: Q8_0, Q8_0: Q8_0, Q4_1: Q8_1}
TYPE_NAME = {F32: "f32", F16: "f16", Q4_0: "q4_0", Q4_1: "q4_1", Q8_0: "q8_0", Q8_1: "q8_1"}
NAME_TYPE = {v: k for k, v in TYPE_NAME.items()}


class OrcTensor(C.Structure):
    _fields_ = [("type", C.c_int32), ("pad_", C.c_int32), ("ne", C.c_int64 * 4),
                ("nb", C.c_int64 * 4), ("data", C.c_void_p)]


def build(force: bool = False) -> str:
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        P, I64, F, I = C.c_void_p, C.c_int64, C.c_float, C.c_int
        T = C.POINTER(OrcTensor)
        sig = {
            "orc_fp32_to_fp16": (C.c_uint16, [F]),
            "orc_fp16_to_fp32": (F, [C.c_uint16]),
            "orc_fp32_to_fp16_row": (None, [P, P, I64]),
            "orc_fp16_to_fp32_row": (None, [P, P, I64]),
            "orc_fill_normal": (None, [P, I64, C.c_uint64, C.c_uint64, F, F]),
            "orc_fill_uniform": (None, [P, I64, C.c_uint64, C.c_uint64, F, F]),
            "orc_quantize_row_q8_0_ref": (None, [P, P, I64]),
            "orc_quantize_row_q8_0_x86": (None, [P, P, I64]),
            "orc_quantize_row_q8_1_ref": (None, [P, P, I64]),
            "orc_quantize_row_q8_1_x86": (None, [P, P, I64]),
            "orc_quantize_row_q4_0_ref": (None, [P, P, I64]),
            "orc_quantize_row_q4_1_ref": (None, [P, P, I64]),
            "orc_quantize_chunk": (I64, [I, P, P, I64, I64, I64]),
            "orc_from_float": (I, [I, I, P, P, I64]),
            "orc_dequantize_row": (I, [I, P, P, I64]),
            "orc_vec_dot": (F, [I, I64, P, P, I]),
            "orc_block_isums": (I, [I, I64, P, P, P]),
            "orc_vec_dot_exact": (C.c_double, [I, I64, P, P]),
            "orc_vec_dot_absterm": (C.c_double, [I, I64, P, P]),
            "orc_mul_mat": (I, [T, T, T, I, I, I]),
            "orc_mul_mat_exact": (I, [T, T, T, P, I, I]),
            "orc_soft_max_ext": (I, [T, T, F, I]),
            "orc_flash_attn_ext": (I, [T, T, T, T, F, F, I]),
            "orc_attn_exact": (I, [T, T, T, T, F, I]),
            "orc_norm_rows": (None, [P, P, I64, I64, F]),
            "orc_gelu_erf": (None, [P, P, I64]),
            "orc_gelu_tanh": (None, [P, P, I64]),
            "orc_hiera_win_part": (None, [P, P, I64, I64, I64, I]),
            "orc_hiera_win_unpart": (None, [P, P, I64, I64, I64, I]),
            "orc_maxpool2": (None, [P, P, I64, I64, I64, I64]),
            "orc_compute_axial_cis": (None, [P, I, I, I, F, F]),
            "orc_sam2_pos_embed": (None, [P, I, I, I, P, I, I, I, P]),
            "orc_apply_rope": (None, [P, P, I64, I64, I64]),
            "orc_win_part": (None, [P, P, I64, I64, I64, I]),
            "orc_win_unpart": (None, [P, P, I64, I64, I64, I]),
            "orc_isa_path": (I, []),
            "orc_set_isa": (None, [I]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def nthreads() -> int:
    """Host threads for oracle work (capped at 16: the host CPU share of one GPU)."""
    return max(1, min(16, os.cpu_count() or 1))


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"] or a.ndim == 0
    return a.ctypes.data


# ---------------------------------------------------------------- inputs
def normal(n: int, seed: int, stream: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().orc_fill_normal(_p(out), n, seed, stream, mean, std)
    return out


def uniform(n: int, seed: int, stream: int, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().orc_fill_uniform(_p(out), n, seed, stream, lo, hi)
    return out


# ---------------------------------------------------------------- quantize
def row_size(t: int, ne0: int) -> int:
    return TYPE_SIZE[t] * (ne0 // BLCK[t])


def quantize_weights(t: int, w: np.ndarray) -> np.ndarray:
    """ggml_quantize_chunk(t, w, ..., imatrix=NULL) -> uint8 [rows, row_size]."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, k = w.shape
    out = np.empty((rows, row_size(t, k)), dtype=np.uint8)
    n = lib().orc_quantize_chunk(t, _p(w), _p(out), 0, rows, k)
    assert n == out.size
    return out


def from_float(t: int, x: np.ndarray, variant: int = ACT_X86) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = x.reshape(-1, x.shape[-1]).shape
    xx = x.reshape(rows, k)
    out = np.empty((rows, row_size(t, k)), dtype=np.uint8)
    for r in range(rows):
        rc = lib().orc_from_float(t, variant, _p(xx[r]), out[r].ctypes.data, k)
        assert rc == 0
    return out


def dequantize(t: int, q: np.ndarray, k: int) -> np.ndarray:
    q = np.ascontiguousarray(q)
    rows = q.shape[0]
    out = np.empty((rows, k), dtype=np.float32)
    for r in range(rows):
        assert lib().orc_dequantize_row(t, q[r].ctypes.data, out[r].ctypes.data, k) == 0
    return out


def fp16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_fp32_to_fp16_row(_p(x), _p(out), x.size)
    return out


# ---------------------------------------------------------------- tensors
def tensor(arr: np.ndarray, t: int, ne, nb=None) -> OrcTensor:
    """orc_tensor over arr's buffer with ggml ne (ne[0] contiguous)."""
    ne = list(ne) + [1] * (4 - len(ne))
    ts = TYPE_SIZE[t]
    if nb is None:
        nb = [ts, row_size(t, ne[0])]
        nb.append(nb[1] * ne[1])
        nb.append(nb[2] * ne[2])
    T = OrcTensor()
    T.type = t
    for i in range(4):
        T.ne[i] = int(ne[i])
        T.nb[i] = int(nb[i])
    T.data = arr.ctypes.data
    T._keep = arr
    return T


def mul_mat(src0_q: np.ndarray, t0: int, K: int, N: int, x: np.ndarray, dims=(1, 1, 1, 1),
            act_variant: int = ACT_X86, order: int = ORDER_X86, exact: bool = False,
            src1_type: int = F32):
    """dst[b3][b2][m][n] = ggml_mul_mat(src0, src1).

    src0_q: uint8/uint16/float32 buffer holding ne02*ne03 stacked [N, row] weights.
    x: src1 [ne13, ne12, M, K] float32 (or float16 bits if src1_type is F16).
    dims: (ne02, ne03, ne12, ne13)."""
    ne02, ne03, ne12, ne13 = dims
    M = x.shape[-2]
    s0 = tensor(src0_q, t0, [K, N, ne02, ne03])
    s1 = tensor(x, src1_type, [K, M, ne12, ne13])
    dst = np.zeros((ne13, ne12, M, N), dtype=np.float32)
    d = tensor(dst, F32, [N, M, ne12, ne13])
    absterm = None
    if exact:
        absterm = np.zeros((ne13 * ne12 * M, N), dtype=np.float32)
        rc = lib().orc_mul_mat_exact(C.byref(s0), C.byref(s1), C.byref(d), _p(absterm), act_variant, nthreads())
    else:
        rc = lib().orc_mul_mat(C.byref(s0), C.byref(s1), C.byref(d), act_variant, order, nthreads())
    if rc != 0:
        raise ValueError(f"orc_mul_mat rc={rc}")
    if exact:
        return dst, absterm.reshape(dst.shape)
    return dst


def soft_max_ext(x: np.ndarray, scale: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    ne = list(x.shape[::-1])
    out = np.empty_like(x)
    rc = lib().orc_soft_max_ext(C.byref(tensor(x, F32, ne)), C.byref(tensor(out, F32, ne)), scale, nthreads())
    assert rc == 0
    return out


def flash_attn_ext(q: OrcTensor, k: OrcTensor, v: OrcTensor, D_v: int, scale: float,
                   softcap: float = 0.0, exact: bool = False) -> np.ndarray:
    """Returns dst [batch, n_q, n_head, Dv] (ggml ne [Dv, n_head, n_q, batch])."""
    nq, nh, nb3 = q.ne[1], q.ne[2], q.ne[3]
    dst = np.zeros((nb3, nq, nh, D_v), dtype=np.float32)
    d = tensor(dst, F32, [D_v, nh, nq, nb3])
    if exact:
        rc = lib().orc_attn_exact(C.byref(q), C.byref(k), C.byref(v), C.byref(d), scale, nthreads())
    else:
        rc = lib().orc_flash_attn_ext(C.byref(q), C.byref(k), C.byref(v), C.byref(d), scale, softcap, nthreads())
    assert rc == 0, rc
    return dst


# ---------------------------------------------------------------- numpy block codecs
def sam2_pos_embed(bkg: np.ndarray, win: np.ndarray, H: int, W: int) -> np.ndarray:
    """bkg [E][bh][bw], win [E][ws][ws] float32 -> [H*W][E] (sam3.cpp:4118-4157)."""
    bkg = np.ascontiguousarray(bkg, dtype=np.float32)
    win = np.ascontiguousarray(win, dtype=np.float32)
    E, bh, bw = bkg.shape
    ws = win.shape[1]
    out = np.empty((H * W, E), dtype=np.float32)
    lib().orc_sam2_pos_embed(_p(bkg), E, bh, bw, _p(win), ws, H, W, _p(out))
    return out


def decode_blocks(t: int, q: np.ndarray, k: int):
    """Independent numpy decoder of the block bytes: (qvals int32 [rows,k], d f32 [rows,nb],
    extra f32 [rows,nb] (m for q4_1, s for q8_1, else zeros))."""
    q = np.ascontiguousarray(q, dtype=np.uint8)
    rows = q.shape[0]
    nb = k // QK
    blk = q.reshape(rows, nb, TYPE_SIZE[t])
    d = blk[:, :, 0:2].copy().view(np.float16).reshape(rows, nb).astype(np.float32)
    extra = np.zeros((rows, nb), dtype=np.float32)
    if t in (Q8_0, Q8_1):
        off = 2 if t == Q8_0 else 4
        if t == Q8_1:
            extra = blk[:, :, 2:4].copy().view(np.float16).reshape(rows, nb).astype(np.float32)
        vals = blk[:, :, off:off + 32].copy().view(np.int8).astype(np.int32)
    else:
        off = 2 if t == Q4_0 else 4
        if t == Q4_1:
            extra = blk[:, :, 2:4].copy().view(np.float16).reshape(rows, nb).astype(np.float32)
        by = blk[:, :, off:off + 16].astype(np.int32)
        vals = np.concatenate([by & 0x0F, by >> 4], axis=2)
        if t == Q4_0:
            vals = vals - 8
    return vals.reshape(rows, k), d, extra
