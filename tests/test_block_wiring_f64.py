"""An independent float64 restatement of the two encoder blocks, written in
torch from the reference's graph code, pinning the wiring of the oracle's
block compositions (oracle/blocks.py, used as the checker of every encoder
parity test):

  * sam3_vit_block_forward (sam3.cpp:3714-3805): LayerNorm eps 1e-5
    (sam3.cpp:1041-1051), ggml_win_part / ggml_win_unpart (window
    py * nw + px, token ly * ws + lx), the qkv columns split as
    [E, 3] (q, k, v), heads as [HD, NH], RoPE on the pairs (x[2i], x[2i+1])
    (sam3_apply_rope, sam3.cpp:3671-3710) with the axial frequencies of
    sam3_compute_axial_cis (sam3.cpp:3559-3590: the first HD/4 pairs along
    x, the next HD/4 along y), softmax(q k^T / sqrt(HD)) v, the projection,
    the residual onto the block input, LayerNorm, fc1, GELU (erf), fc2, the
    second residual;
  * sam2_hiera_block_forward (sam3.cpp:4299-4461): LayerNorm eps 1e-6,
    the shortcut (dim_proj of the normed input, 2x2 max pool under a q
    stride), sam2_window_partition with zero padding and the H-major window
    order n = wh + ww * nW_h (sam3.cpp:4194-4232, restated here as the
    reference's own reshape / permute sequence), Q pooled inside each
    window, the unpartition at ws // 2 with its own padding and crop
    (sam3.cpp:4234-4281, 4420-4438), and ggml_gelu's fp16 table form in
    the MLP.

The weights are F16, so a MUL_MAT is the reference's F16 semantics (the
activations rounded to fp16 as ggml_fp32_to_fp16_row does, products of two
halves exact; sam3.cpp:6640-6675) evaluated in float64 here and in fp32 by
the oracle.  The two agree to rounding (measured max 4e-5 to 6e-4 on outputs
up to 10; bar 2e-3).  The qkv weights are drawn large enough that the
attention is far from uniform, and each planted wiring mistake in the
restatement (q and k swapped, k and v swapped, the RoPE pairs shifted by one
dimension, the residual taken from the normed input, the tokens of each ViT
window transposed, the Hiera windows cut in raster order, the pooled query
replaced by a strided one, the dim_proj shortcut taken from the raw input)
moves the output by more than 25 times the bar (measured 1.2 to 11), so the
comparison would catch the same mistake in the oracle.  The GELU forms
(erf for the ViT, the fp16 tanh table for Hiera) differ from each other by
about 1e-3 here, below what a block comparison resolves; they are pinned as
functions by the oracle's node tests.  CPU only."""
import math
import types

import numpy as np
import pytest
import torch

from block_refs import axial_cis, hiera_block_ref, vit_block_ref

F64 = torch.float64
BAR = 2e-3
MUTATION_FACTOR = 25.0


def f16_act(t):
    """An fp32 activation rounded to fp16 (ggml_fp32_to_fp16_row), as float64."""
    return t.to(torch.float32).to(torch.float16).to(F64)


def linear(x, w16, b):
    """ggml_mul_mat with F16 weights [N][K] plus the bias: exact f16 x f16 products."""
    return f16_act(x) @ w16.T + b


def layer_norm(x, w, b, eps):
    mu = x.mean(-1, keepdim=True)
    var = ((x - mu) ** 2).mean(-1, keepdim=True)
    return (x - mu) / torch.sqrt(var + eps) * w + b


def axial_freqs(hd, end, scale, theta=10000.0):
    """cos, sin [end * end][hd / 2]: pair j < hd/4 rotates by t_x * f_j, pair hd/4 + j by
    t_y * f_j, f_j = theta^(-4j / hd), token t = y * end + x."""
    q = hd // 4
    f = 1.0 / theta ** (torch.arange(q, dtype=F64) * 4.0 / hd)
    t = torch.arange(end * end)
    tx = (t % end).to(F64) * scale
    ty = torch.div(t, end, rounding_mode="floor").to(F64) * scale
    ang = torch.cat([tx[:, None] * f, ty[:, None] * f], dim=1)
    return torch.cos(ang), torch.sin(ang)


def rope(x, cos, sin, shift=False):
    """Complex rotation of (x[2i], x[2i+1]) by (cos_i, sin_i) over the last dim; shift
    (a planted mistake) pairs (x[2i+1], x[2i+2]) instead."""
    if shift:
        x = torch.roll(x, -1, dims=-1)
    xr, xi = x[..., 0::2], x[..., 1::2]
    out = torch.empty_like(x)
    out[..., 0::2] = xr * cos - xi * sin
    out[..., 1::2] = xr * sin + xi * cos
    return torch.roll(out, 1, dims=-1) if shift else out


def attention(q, k, v, hd):
    return torch.softmax(q @ k.transpose(-1, -2) / math.sqrt(hd), dim=-1) @ v


def maxpool2(x):
    """2x2 / stride-2 max pool over the two dims before the channels of [..., H, W, C]."""
    *lead, H, W, C = x.shape
    return x.reshape(*lead, H // 2, 2, W // 2, 2, C).amax(dim=(-4, -2))


def gelu_tanh_table(x):
    """ggml_gelu with the fp16 table: 0 below -10, x above 10, else f16(gelu(f16(x)))."""
    h = f16_act(x)
    g = 0.5 * h * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * h * (1.0 + 0.044715 * h * h)))
    g = f16_act(g)
    return torch.where(x <= -10.0, torch.zeros_like(x), torch.where(x >= 10.0, x, g))


def vit_block_f64(x, W, v, E, NH, grid, ws, rope_end, rope_scale, mut=()):
    HD = E // NH
    img = x.reshape(grid, grid, E)  # image rows h * grid + w
    xn = layer_norm(img, v["norm1_w"], v["norm1_b"], 1e-5)
    if ws:
        nw = grid // ws
        order = (0, 2, 3, 1, 4) if "window_transpose" in mut else (0, 2, 1, 3, 4)
        win = xn.reshape(nw, ws, nw, ws, E).permute(*order).reshape(nw * nw, ws * ws, E)
    else:
        win = xn.reshape(1, grid * grid, E)
    qkv = linear(win, W["qkv"], v["qkv_b"])
    q, k, vv = qkv.split(E, dim=-1)
    if "swap_qk" in mut:
        q, k = k, q
    if "swap_kv" in mut:
        k, vv = vv, k
    heads = lambda t: t.reshape(t.shape[0], t.shape[1], NH, HD).transpose(1, 2)
    q, k, vv = heads(q), heads(k), heads(vv)
    cos, sin = axial_freqs(HD, rope_end, rope_scale)
    q, k = rope(q, cos, sin, "rope_shift" in mut), rope(k, cos, sin, "rope_shift" in mut)
    att = attention(q, k, vv, HD).transpose(1, 2).reshape(win.shape[0], win.shape[1], E)
    p = linear(att, W["proj"], v["proj_b"])
    if ws:
        inv = (0, 3, 1, 2, 4) if "window_transpose" in mut else (0, 2, 1, 3, 4)
        p = p.reshape(nw, nw, ws, ws, E).permute(*inv).reshape(grid, grid, E)
    else:
        p = p.reshape(grid, grid, E)
    r = (xn if "residual_from_norm" in mut else img) + p
    h = linear(layer_norm(r, v["norm2_w"], v["norm2_b"], 1e-5), W["fc1"], v["fc1_b"])
    h = 0.5 * h * (1.0 + torch.erf(h / math.sqrt(2.0)))
    return (r + linear(h, W["fc2"], v["fc2_b"])).reshape(grid * grid, E)


def sam2_partition(x, ws, mut=()):
    """sam2_window_partition as the reference's reshape / permute sequence, in torch's
    reversed dims ([H][W][C] for ggml [C, W, H]): pad, [Hp][nW_w][ws*C] -> permute ->
    [nW_w][Hp][ws*C] -> [nW_w][nW_h][ws][ws*C] -> [nW][ws][ws][C]."""
    H, W, C = x.shape
    Hp, Wp = -(-H // ws) * ws, -(-W // ws) * ws
    xp = torch.zeros((Hp, Wp, C), dtype=x.dtype)
    xp[:H, :W] = x
    r1 = xp.reshape(Hp, Wp // ws, ws * C)
    c1 = (r1 if "window_order" in mut else r1.permute(1, 0, 2)).contiguous()
    return c1.reshape(-1, ws, ws, C).reshape(-1, ws * ws, C), (Hp, Wp)


def sam2_unpartition(x, ws, pad_hw, H, W, mut=()):
    """sam2_window_unpartition: [nW][ws*ws][C] -> [nW_w][Hp][ws*C] -> permute ->
    [Hp][nW_w][ws*C] -> [Hp][Wp][C], cropped to [H][W][C]."""
    Hp, Wp = pad_hw
    C = x.shape[-1]
    r2 = x.reshape(Wp // ws, Hp, ws * C) if "window_order" not in mut else x.reshape(Hp, Wp // ws, ws * C)
    c1 = (r2.permute(1, 0, 2) if "window_order" not in mut else r2).contiguous()
    return c1.reshape(Hp, Wp, C)[:H, :W]


def hiera_block_f64(x, W, v, Cin, Cout, NH, S, ws, qs, mut=()):
    HD = Cout // NH
    img = x.reshape(S, S, Cin)
    xn = layer_norm(img, v["norm1_w"], v["norm1_b"], 1e-6)
    if Cin != Cout:
        sc = linear(img if "residual_from_input" in mut else xn, W["dim_proj"], v["dim_proj_b"])
        sc = maxpool2(sc) if qs else sc
    else:
        sc = maxpool2(img) if qs else img
    if ws:
        win, pad_hw = sam2_partition(xn, ws, mut)
        side = ws
    else:
        win, pad_hw, side = xn.reshape(1, S * S, Cin), (S, S), S
    qkv = linear(win, W["qkv"], v["qkv_b"])
    q, k, vv = qkv.split(Cout, dim=-1)
    if "swap_qk" in mut:
        q, k = k, q
    nq_side = side
    if qs and "no_qpool" not in mut:
        q = maxpool2(q.reshape(q.shape[0], side, side, Cout)).reshape(q.shape[0], -1, Cout)
        nq_side = side // 2
    elif qs:  # the planted mistake: every other query kept instead of the pooled maximum
        q = q.reshape(q.shape[0], side, side, Cout)[:, ::2, ::2].reshape(q.shape[0], -1, Cout)
        nq_side = side // 2
    heads = lambda t: t.reshape(t.shape[0], t.shape[1], NH, HD).transpose(1, 2)
    att = attention(heads(q), heads(k), heads(vv), HD).transpose(1, 2).reshape(q.shape[0], -1, Cout)
    p = linear(att, W["proj"], v["proj_b"])
    T = S // 2 if qs else S
    if ws:
        wso = ws // 2 if qs else ws
        pad = (wso - T % wso) % wso
        p = sam2_unpartition(p, wso, (T + pad, T + pad) if qs else pad_hw, T, T, mut)
    else:
        p = p.reshape(nq_side, nq_side, Cout)
    res1 = sc + p
    h = linear(layer_norm(res1, v["norm2_w"], v["norm2_b"], 1e-6), W["fc1"], v["fc1_b"])
    h = gelu_tanh_table(h)
    return (res1 + linear(h, W["fc2"], v["fc2_b"])).reshape(T * T, Cout)


def _weights(orc, shapes, vecs, seed, std):
    host, W = {}, {}
    for i, (name, (N, K)) in enumerate(shapes.items()):
        w16 = (orc.normal(N * K, seed, 10 + i, std=std.get(name, 0.05)).reshape(N, K)).astype(np.float16)
        host[name] = (w16.view(np.uint16), N, K)
        W[name] = torch.from_numpy(w16.astype(np.float64))
    vec, v = {}, {}
    for i, (name, n, s, m) in enumerate(vecs):
        a = orc.normal(n, seed, 40 + i) * np.float32(s) + np.float32(m)
        vec[name] = a
        v[name] = torch.from_numpy(a.astype(np.float64))
    return host, vec, W, v


def _check(name, ref, restated, mutated):
    d = float(np.abs(ref.astype(np.float64) - restated.numpy()).max())
    scale = float(np.abs(restated.numpy()).max())
    print(f"{name}: max |oracle - float64 restatement| {d:.2e} (outputs up to {scale:.2f})", flush=True)
    assert d <= BAR, f"{name}: oracle and restatement differ by {d:.3e}"
    for mname, out in mutated.items():
        dm = float(np.abs(ref.astype(np.float64) - out.numpy()).max())
        print(f"  planted '{mname}': {dm:.2e}", flush=True)
        assert dm >= MUTATION_FACTOR * BAR, f"{name}: planted '{mname}' moves the output by only {dm:.3e}"


@pytest.mark.parametrize("ws", [4, 0])
def test_vit_block_wiring(orc, ws):
    E, NH, MLP, grid = 64, 2, 128, 8
    shapes = {"qkv": (3 * E, E), "proj": (E, E), "fc1": (MLP, E), "fc2": (E, MLP)}
    vecs = [("norm1_w", E, 0.2, 1.0), ("norm1_b", E, 0.1, 0.0), ("qkv_b", 3 * E, 0.05, 0.0), ("proj_b", E, 0.05, 0.0),
            ("norm2_w", E, 0.2, 1.0), ("norm2_b", E, 0.1, 0.0), ("fc1_b", MLP, 0.05, 0.0), ("fc2_b", E, 0.05, 0.0)]
    host, vec, W, v = _weights(orc, shapes, vecs, seed=21 + ws, std={"qkv": 0.25, "proj": 0.1, "fc1": 0.1, "fc2": 0.1})
    x = orc.normal(grid * grid * E, 22 + ws, 1).reshape(grid * grid, E)
    end, scale = (ws, 1.0) if ws else (grid, 0.5)
    freqs = axial_cis(orc, E // NH, end, scale)
    ref = vit_block_ref(orc, orc.F16, x, host, vec, E, NH, MLP, grid, ws, freqs, False)
    xt = torch.from_numpy(x.astype(np.float64))
    run = lambda mut=(): vit_block_f64(xt, W, v, E, NH, grid, ws, end, scale, mut)
    muts = ["swap_qk", "swap_kv", "rope_shift", "residual_from_norm"] + (["window_transpose"] if ws else [])
    _check(f"ViT block ws={ws}", ref, run(), {m: run((m,)) for m in muts})


@pytest.mark.parametrize("kind", ["windowed", "windowed_padded", "q_stride", "global"])
def test_hiera_block_wiring(orc, kind):
    Cin, Cout, NH, S, ws, qs = {"windowed": (32, 32, 1, 8, 4, 0), "windowed_padded": (32, 32, 1, 6, 4, 0),
                                "q_stride": (32, 64, 2, 8, 4, 1), "global": (64, 64, 2, 8, 0, 0)}[kind]
    shapes = {"qkv": (3 * Cout, Cin), "proj": (Cout, Cout), "fc1": (4 * Cout, Cout), "fc2": (Cout, 4 * Cout)}
    vecs = [("norm1_w", Cin, 0.2, 1.0), ("norm1_b", Cin, 0.1, 0.0), ("qkv_b", 3 * Cout, 0.05, 0.0),
            ("proj_b", Cout, 0.05, 0.0), ("norm2_w", Cout, 0.2, 1.0), ("norm2_b", Cout, 0.1, 0.0),
            ("fc1_b", 4 * Cout, 0.05, 0.0), ("fc2_b", Cout, 0.05, 0.0)]
    if Cin != Cout:
        shapes["dim_proj"] = (Cout, Cin)
        vecs.append(("dim_proj_b", Cout, 0.05, 0.0))
    host, vec, W, v = _weights(orc, shapes, vecs, seed=31 + len(kind), std={"qkv": 0.3, "proj": 0.15, "fc1": 0.1,
                                                                              "fc2": 0.1, "dim_proj": 0.15})
    x = orc.normal(S * S * Cin, 32 + len(kind), 1).reshape(S * S, Cin)
    info = types.SimpleNamespace(dim_in=Cin, dim_out=Cout, num_heads=NH, window_size=ws, q_stride=qs)
    _, ref = hiera_block_ref(orc, orc.F16, x, info, host, vec, S, False)
    xt = torch.from_numpy(x.astype(np.float64))
    run = lambda mut=(): hiera_block_f64(xt, W, v, Cin, Cout, NH, S, ws, qs, mut)
    muts = ["swap_qk"] + (["window_order"] if ws else []) + (["no_qpool"] if qs else []) + \
           (["residual_from_input"] if Cin != Cout else [])
    _check(f"Hiera block {kind}", ref, run(), {m: run((m,)) for m in muts})
