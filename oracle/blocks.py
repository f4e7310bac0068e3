"""Oracle compositions of the two encoder blocks: sam3_vit_block_forward
(sam3.cpp:3714-3805) and sam2_hiera_block_forward (sam3.cpp:4299-4461)
built from the oracle's ggml node restatements.

TEST INFRASTRUCTURE ONLY, like the rest of oracle/: used by the GPU parity
tests (as the checker) and by the cpu_baseline leg of bench.py (the encoder
block timed on the host cores); the product library never uses it.

Both take an optional query selection: a block's output row depends on
every token only through the keys and values of its attention, so the
oracle can evaluate a subset of output rows exactly (LayerNorm and the qkv
GEMM over all tokens; attention, projection, residual and MLP for the chosen
query rows only).  The full-size parity tests use this to keep the CPU side
at a few seconds; tests/test_oracle_blocks.py holds the sampled form equal
to the full composition row for row.
"""
import ctypes as C

import numpy as np


# ---------------------------------------------------------------- ggml node restatements
def ln_ref(orc, x, w, b, eps=1e-5):
    """sam3_layer_norm: ggml_norm, ggml_mul(w), ggml_add(b) (sam3.cpp:1041-1051)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    orc.lib().orc_norm_rows(x.ctypes.data, y.ctypes.data, x.shape[0], x.shape[1], C.c_float(eps))
    if w is not None:
        y = (y * w).astype(np.float32)
    if b is not None:
        y = (y + b).astype(np.float32)
    return y


def win_part(orc, x, grid, ws):
    """ggml_win_part (sam3.cpp:3734): image order -> window order."""
    E = x.shape[1]
    out = np.empty_like(x)
    orc.lib().orc_win_part(np.ascontiguousarray(x).ctypes.data, out.ctypes.data, E, grid, grid, ws)
    return out


def win_unpart(orc, x, grid, ws):
    """ggml_win_unpart (sam3.cpp:3788): window order -> image order."""
    E = x.shape[1]
    out = np.empty_like(x)
    orc.lib().orc_win_unpart(np.ascontiguousarray(x).ctypes.data, out.ctypes.data, E, grid, grid, ws)
    return out


def win_rows(orc, grid, ws):
    """perm[r] = image row of window-order row r (ggml_win_part of the row index)."""
    idx = np.repeat(np.arange(grid * grid, dtype=np.float32)[:, None], 4, axis=1)
    return win_part(orc, idx, grid, ws)[:, 0].astype(np.int64)


def axial_cis(orc, hd, end, scale):
    """sam3_compute_axial_cis (sam3.cpp:3559-3590): [end*end][hd/2][2] (cos, sin)."""
    out = np.empty(end * end * hd, dtype=np.float32)
    orc.lib().orc_compute_axial_cis(out.ctypes.data, hd, end, end, C.c_float(10000.0), C.c_float(scale))
    return out


def rope_ref(orc, x, freqs, hd, n):
    """x [rows3][n][hd] float32, RoPE in place (sam3.cpp:3671-3710)."""
    x = np.ascontiguousarray(x, dtype=np.float32).copy()
    orc.lib().orc_apply_rope(x.ctypes.data, freqs.ctypes.data, hd, n, x.size // (n * hd))
    return x


def gelu_ref(orc, x):
    """ggml_gelu_erf."""
    y = np.empty_like(x)
    orc.lib().orc_gelu_erf(np.ascontiguousarray(x).ctypes.data, y.ctypes.data, x.size)
    return y


def gelu_tanh(orc, x):
    """ggml_gelu (fp16 table form)."""
    y = np.empty_like(x)
    orc.lib().orc_gelu_tanh(np.ascontiguousarray(x).ctypes.data, y.ctypes.data, x.size)
    return y


def hiera_win_part(orc, x, S, C_, ws):
    """sam2_window_partition (sam3.cpp:4194-4230), zero padding."""
    nw = (-(-S // ws)) ** 2
    out = np.empty((nw * ws * ws, C_), dtype=np.float32)
    orc.lib().orc_hiera_win_part(np.ascontiguousarray(x).ctypes.data, out.ctypes.data, C_, S, S, ws)
    return out


def hiera_win_unpart(orc, x, S, C_, ws):
    """sam2_window_unpartition with crop (sam3.cpp:4232-4281)."""
    out = np.empty((S * S, C_), dtype=np.float32)
    orc.lib().orc_hiera_win_unpart(np.ascontiguousarray(x).ctypes.data, out.ctypes.data, C_, S, S, ws)
    return out


def maxpool2(orc, x, C_, W, H, B=1):
    """2x2 / stride-2 max pool over B maps of [H][W][C_]."""
    out = np.empty((B * (H // 2) * (W // 2), C_), dtype=np.float32)
    orc.lib().orc_maxpool2(np.ascontiguousarray(x).ctypes.data, out.ctypes.data, C_, W, H, B)
    return out


def _mm(orc, t, host, name, x):
    q, N, K = host[name]
    return orc.mul_mat(q, t, K, N, np.ascontiguousarray(x, dtype=np.float32)).reshape(-1, N)


def _attention(orc, Q, K, V, HD, f16_attn):
    """ggml_flash_attn_ext(Q, K, V, scale 1/sqrt(HD)) over [B][NH][n][HD] arrays.
    f16_attn: Q/K/V rounded to fp16 first (the GPU's operand precision),
    evaluated exactly; otherwise ggml-cpu's F32 attention."""
    B, NH, nq, _ = Q.shape
    nkv = K.shape[2]
    if f16_attn:
        Q, K, V = (np.ascontiguousarray(a.astype(np.float16)) for a in (Q, K, V))
        tt = orc.F16
    else:
        Q, K, V = (np.ascontiguousarray(a, dtype=np.float32) for a in (Q, K, V))
        tt = orc.F32
    out = orc.flash_attn_ext(orc.tensor(Q, tt, [HD, nq, NH, B]), orc.tensor(K, tt, [HD, nkv, NH, B]),
                             orc.tensor(V, tt, [HD, nkv, NH, B]), HD, 1.0 / np.sqrt(HD), exact=f16_attn)
    return out  # [B][nq][NH][HD]


# ---------------------------------------------------------------- SAM3 ViT block
def vit_qkv(orc, t, x, host, vec, E, NH, grid, ws, freqs):
    """The attention operands of sam3_vit_block_forward: LN1, win_part, qkv
    GEMM + bias, split, RoPE on Q and K.  Returns Q, K, V [B][NH][N][HD]."""
    HD = E // NH
    M = grid * grid
    N = ws * ws if ws else M
    B = M // N
    xn = ln_ref(orc, x, vec["norm1_w"], vec["norm1_b"])
    if ws:
        xn = win_part(orc, xn, grid, ws)
    qkv = (_mm(orc, t, host, "qkv", xn) + vec["qkv_b"]).astype(np.float32)
    parts = [np.ascontiguousarray(qkv[:, i * E:(i + 1) * E].reshape(B, N, NH, HD).transpose(0, 2, 1, 3))
             for i in range(3)]
    Q = rope_ref(orc, parts[0], freqs, HD, N).reshape(B, NH, N, HD) if freqs is not None else parts[0]
    K = rope_ref(orc, parts[1], freqs, HD, N).reshape(B, NH, N, HD) if freqs is not None else parts[1]
    return Q, K, parts[2]


def vit_block_rows(orc, t, x, host, vec, E, NH, MLP, grid, ws, freqs, f16_attn, qsel=None, qkv=None):
    """sam3_vit_block_forward (sam3.cpp:3714-3805) for the query positions
    qsel (indices inside every attention batch; all when None).  Returns
    (image rows, their output rows).  qkv: vit_qkv's result, if computed."""
    HD = E // NH
    M = grid * grid
    N = ws * ws if ws else M
    B = M // N
    Q, K, V = qkv if qkv is not None else vit_qkv(orc, t, x, host, vec, E, NH, grid, ws, freqs)
    qsel = np.arange(N) if qsel is None else np.asarray(qsel)
    att = _attention(orc, np.ascontiguousarray(Q[:, :, qsel]), K, V, HD, f16_attn).reshape(B * len(qsel), E)
    p = (_mm(orc, t, host, "proj", att) + vec["proj_b"]).astype(np.float32)
    wrows = (np.arange(B)[:, None] * N + qsel[None, :]).reshape(-1)
    rows = win_rows(orc, grid, ws)[wrows] if ws else wrows
    xr = (x[rows] + p).astype(np.float32)  # ggml_win_unpart + residual add
    xn = ln_ref(orc, xr, vec["norm2_w"], vec["norm2_b"])
    h = gelu_ref(orc, (_mm(orc, t, host, "fc1", xn) + vec["fc1_b"]).astype(np.float32))
    f = _mm(orc, t, host, "fc2", h)
    return rows, (xr + (f + vec["fc2_b"]).astype(np.float32)).astype(np.float32)


def vit_block_ref(orc, t, x, host, vec, E, NH, MLP, grid, ws, freqs, f16_attn):
    """The whole block's output [grid*grid][E] in image order."""
    rows, out = vit_block_rows(orc, t, x, host, vec, E, NH, MLP, grid, ws, freqs, f16_attn)
    full = np.empty_like(x)
    full[rows] = out
    return full


# ---------------------------------------------------------------- SAM2 Hiera block
def hiera_block_ref(orc, t, x, info, host, vec, S, f16_attn, qsel=None):
    """sam2_hiera_block_forward (sam3.cpp:4299-4461) from oracle pieces;
    x [S*S][Cin].  qsel (global blocks without Q pooling only) evaluates those
    token rows; returns (rows, output rows).  Without qsel rows = all."""
    Cin, Cout, NH, ws, qs = info.dim_in, info.dim_out, info.num_heads, info.window_size, info.q_stride
    HD = Cout // NH
    S2 = S // 2 if qs else S
    if qsel is not None:
        assert ws == 0 and not qs and Cin == Cout, "row selection needs a global block without pooling"
    normed = ln_ref(orc, x, vec["norm1_w"], vec["norm1_b"], eps=1e-6)
    if Cin != Cout:
        sc = (_mm(orc, t, host, "dim_proj", normed) + vec["dim_proj_b"]).astype(np.float32)
        if qs:
            sc = maxpool2(orc, sc, Cout, S, S)
    elif qs:
        sc = maxpool2(orc, x, Cout, S, S)
    else:
        sc = x
    if ws > 0:
        att_in = hiera_win_part(orc, normed, S, Cin, ws)
        nW, Nkv = (-(-S // ws)) ** 2, ws * ws
    else:
        att_in, nW, Nkv = normed, 1, S * S
    qkv = (_mm(orc, t, host, "qkv", att_in) + vec["qkv_b"]).astype(np.float32)
    q, k, v = (np.ascontiguousarray(qkv[:, i * Cout:(i + 1) * Cout]) for i in range(3))
    if qs:
        q = maxpool2(orc, q, Cout, ws, ws, nW)
        Nq = (ws // 2) ** 2
    else:
        Nq = Nkv
    Q = np.ascontiguousarray(q.reshape(nW, Nq, NH, HD).transpose(0, 2, 1, 3))
    K = np.ascontiguousarray(k.reshape(nW, Nkv, NH, HD).transpose(0, 2, 1, 3))
    V = np.ascontiguousarray(v.reshape(nW, Nkv, NH, HD).transpose(0, 2, 1, 3))
    rows = np.arange(S2 * S2) if qsel is None else np.asarray(qsel)
    if qsel is not None:
        Q = np.ascontiguousarray(Q[:, :, rows])
    att = _attention(orc, Q, K, V, HD, f16_attn).reshape(-1, Cout)
    p = (_mm(orc, t, host, "proj", att) + vec["proj_b"]).astype(np.float32)
    if ws > 0:
        p = hiera_win_unpart(orc, p, S2, Cout, ws // 2 if qs else ws)
    res1 = (sc[rows] + p).astype(np.float32)
    n2 = ln_ref(orc, res1, vec["norm2_w"], vec["norm2_b"], eps=1e-6)
    h = gelu_tanh(orc, (_mm(orc, t, host, "fc1", n2) + vec["fc1_b"]).astype(np.float32))
    f = (_mm(orc, t, host, "fc2", h) + vec["fc2_b"]).astype(np.float32)
    return rows, (res1 + f).astype(np.float32)
