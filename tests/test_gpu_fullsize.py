"""Full-size parity of both image encoders against the oracle.

SAM3 ViT at 1008x1008 (sam3.cpp:3714-3853): E = 1024, a 72x72 token grid,
16 heads of 64, MLP 4736, windows of 24x24, global blocks 7/15/23/31.
- One windowed and one global block, Q8_0 and Q4_0 weights, on N(0,1)
  activations.
- The 32-block encoder (mi355_vit_encode from a U(0,1) image): the prefix is
  compared with the oracle; the blocks run one by one through
  mi355_vit_block_forward must reproduce the encoder's output bit for bit;
  blocks 0, 7 (global) and 31 are each compared with the oracle run on that
  block's own GPU input (stage isolation as in the reference's
  tests/test_metal_block_stage_compare.cpp:245-271).

SAM2.1 Hiera-tiny at 1024x1024 (sam3.cpp:4299-4535): blocks 0 and 1 at
S = 256 (65536 tokens: the K = 96 projections take the skinny kernel for the
block types), the global block 5 at S = 64, F16 and Q4_0; and the whole
backbone, every block compared with the oracle on its own GPU input.

The oracle evaluates sampled query rows (tests/block_refs.py; the sampled
form equals the full composition row for row, tests/test_oracle_blocks.py),
twice: with the fp16-rounded Q/K/V the GPU attention uses (exact arithmetic;
ggml's GPU backends also convert F32 K/V to F16 for FLASH_ATTN_EXT) and with
ggml-cpu's F32 attention.  At these sizes the two oracle runs themselves
differ by up to 1.4e-2 max / 2.3e-3 RMS (ViT, Q8_0) and 3.6e-2 / 6e-3
(Hiera, Q4_0): any difference in the attention output's last bits flips
some activation-quantization roundings downstream, and each flip moves the
outputs of its row by about d_a * |w| ~ 1e-3.  That spread is the noise
floor of two legitimate implementations, so the bars are stated against it:
- |gpu - oracle| (each oracle run): max <= max(1e-2, 1.5 * spread max) (1e-2
  is the reference's own CPU-vs-GPU block bound,
  tests/test_metal_overhead.cpp:240-246; the max of ~10^5-10^6 elements
  varies by ~15% between noise realisations) and RMS <= max(5e-4, 1.25 *
  spread RMS);
- no systematic error: flips are symmetric, so every column mean and every
  row mean of (gpu - oracle) stays within 6 standard errors of zero
  (6 * that line's RMS / sqrt(count)).  A missing bias, a wrong row map or a scale
  error shifts a whole column or row and fails this at once.
- The prefix: max 1e-4 after ln_pre (F32 patch GEMM rounding only).
"""
import ctypes as C

import numpy as np
import pytest
import torch

from block_refs import axial_cis, block_bars, hiera_block_ref, ln_ref, vit_block_rows, vit_qkv
from gpu_helpers import dev

pytestmark = pytest.mark.gpu

E, NH, MLP, GRID, WS, P, PG = 1024, 16, 4736, 72, 24, 14, 24
HD = E // NH
GLOBAL_BLOCKS = (7, 15, 23, 31)


def _p(t):
    return C.c_void_p(t.data_ptr())


def _hp(mi):
    hp = mi.VitHparams()
    hp.embed_dim, hp.num_heads, hp.mlp_dim, hp.window_size = E, NH, MLP, WS
    hp.grid, hp.patch_size, hp.pos_grid, hp.eps = GRID, P, PG, 1e-5
    return hp


def _vit_block_weights(mi, orc, t, seed, is_global, freqs_dev):
    shapes = {"qkv": (3 * E, E), "proj": (E, E), "fc1": (MLP, E), "fc2": (E, MLP)}
    host, keep = {}, []
    blk = mi.VitBlock()
    for i, (name, (N, K)) in enumerate(shapes.items()):
        w = orc.normal(N * K, seed, 10 + i, std=0.02).reshape(N, K)
        q = w.astype(np.float16).view(np.uint16) if t == orc.F16 else orc.quantize_weights(t, w)
        host[name] = (q, N, K)
        d = dev(q.view(np.uint8))
        keep.append(d)
        setattr(blk, name + "_w", mi.from_torch(d, t, [K, N]))
    vec = {}
    for i, (name, n, s, m) in enumerate([("norm1_w", E, 0.2, 1.0), ("norm1_b", E, 0.1, 0.0), ("qkv_b", 3 * E, 0.05, 0.0),
                                          ("proj_b", E, 0.05, 0.0), ("norm2_w", E, 0.2, 1.0), ("norm2_b", E, 0.1, 0.0),
                                          ("fc1_b", MLP, 0.05, 0.0), ("fc2_b", E, 0.05, 0.0)]):
        vec[name] = orc.normal(n, seed, 20 + i) * np.float32(s) + np.float32(m)
        d = dev(vec[name])
        keep.append(d)
        setattr(blk, name, d.data_ptr())
    blk.freqs_cis = freqs_dev.data_ptr()
    blk.is_global = is_global
    return blk, host, vec, keep


def _qsel(is_global, seed):
    """Query positions the oracle evaluates: 64 per 24x24 window (576 rows), or
    576 of the 5184 global tokens; always including the first and last."""
    rng = np.random.default_rng(seed)
    n, k = (GRID * GRID, 576) if is_global else (WS * WS, 64)
    sel = rng.choice(np.arange(1, n - 1), size=k - 2, replace=False)
    return np.sort(np.concatenate([[0, n - 1], sel]))


def _check_vit_block(orc, t, x_in, got, host, vec, is_global, freqs, seed, what):
    qsel = _qsel(is_global, seed)
    ws = 0 if is_global else WS
    qkv = vit_qkv(orc, t, x_in, host, vec, E, NH, GRID, ws, freqs)
    rows, ref16 = vit_block_rows(orc, t, x_in, host, vec, E, NH, MLP, GRID, ws, freqs, True, qsel=qsel, qkv=qkv)
    _, ref32 = vit_block_rows(orc, t, x_in, host, vec, E, NH, MLP, GRID, ws, freqs, False, qsel=qsel, qkv=qkv)
    assert np.isfinite(got).all(), what
    sp_max, sp_rms = block_bars(got[rows], ref16, ref32, what)
    worst = max(float(np.abs(got[rows] - ref16).max()), float(np.abs(got[rows] - ref32).max()))
    return sp_max, sp_rms, worst


def _freqs(orc, is_global):
    # window tables: 24x24 at scale 1; global: the 72x72 grid at scale 24/72 (sam3.cpp:3559-3590)
    return axial_cis(orc, HD, GRID, WS / GRID) if is_global else axial_cis(orc, HD, WS, 1.0)


@pytest.mark.parametrize("is_global", [0, 1])
@pytest.mark.parametrize("tname", ["q8_0", "q4_0", "f16"])
def test_vit_block_full(mi, ctx, orc, is_global, tname):
    """F16 weights (no activation quantization, so no rounding flips): held to the
    reference's own CPU-vs-GPU block bound, max |diff| < 1e-2
    (tests/test_metal_overhead.cpp:240-246), against both oracle runs."""
    t = orc.NAME_TYPE[tname]
    freqs = _freqs(orc, is_global)
    fd = dev(freqs)
    blk, host, vec, _keep = _vit_block_weights(mi, orc, t, 70 + is_global, is_global, fd)
    x0 = orc.normal(GRID * GRID * E, 71, 1).reshape(GRID * GRID, E)
    x = dev(x0)
    print(f"vit block E={E} grid={GRID} {tname} global={is_global}", flush=True)
    ctx.vit_block_forward(_hp(mi), blk, _p(x))
    ctx.synchronize()
    spread = _check_vit_block(orc, t, x0, x.cpu().numpy(), host, vec, is_global, freqs, 72 + is_global,
                              f"vit block {tname} global={is_global}")
    if t == orc.F16:
        assert spread[2] < 1e-2, f"F16 block max diff {spread[2]:.3e} >= 1e-2"


@pytest.mark.parametrize("tname", ["q8_0", "q4_0"])
def test_vit_encoder_stage_isolation(mi, ctx, orc, tname):
    t = orc.NAME_TYPE[tname]
    hp = _hp(mi)
    S = GRID * P
    img = orc.uniform(3 * S * S, 80, 1).reshape(3, S, S)
    pw = orc.normal(E * 3 * P * P, 80, 2, std=0.02).reshape(E, 3, P, P)  # ggml [P, P, 3, E]
    pos = orc.normal(PG * PG * E, 80, 3).reshape(PG * PG, E)
    lw = orc.normal(E, 80, 4) * np.float32(0.2) + np.float32(1.0)
    lb = orc.normal(E, 80, 5) * np.float32(0.1)
    fw, fg = _freqs(orc, 0), _freqs(orc, 1)
    fwd, fgd = dev(fw), dev(fg)
    check = (0, 7, 31)
    blocks, hosts, keep = [], {}, []
    for i in range(32):
        g = int(i in GLOBAL_BLOCKS)
        blk, host, vec, k = _vit_block_weights(mi, orc, t, 100 + i, g, fgd if g else fwd)
        blocks.append(blk)
        keep.append(k)
        if i in check:
            hosts[i] = (host, vec)
    imgd, pwd, posd, lwd, lbd = dev(img), dev(pw), dev(pos), dev(lw), dev(lb)
    patch = mi.from_torch(pwd, mi.F32, [P, P, 3, E])
    print(f"vit encoder {tname}: 32 blocks at {S}x{S}", flush=True)
    x_enc = torch.empty((GRID * GRID, E), dtype=torch.float32, device="cuda")
    ctx.vit_encode(hp, _p(imgd), patch, _p(posd), _p(lwd), _p(lbd), blocks, _p(x_enc))
    x = torch.empty_like(x_enc)
    ctx.vit_prefix(hp, _p(imgd), patch, _p(posd), _p(lwd), _p(lbd), _p(x))
    ctx.synchronize()
    # prefix: im2col + F32 mul_mat (ggml_conv_2d_sk_p0) + tiled pos_embed + ln_pre, on sampled rows
    rows = np.sort(np.random.default_rng(81).choice(GRID * GRID, 512, replace=False))
    cols = img.reshape(3, GRID, P, GRID, P).transpose(1, 3, 0, 2, 4).reshape(GRID * GRID, 3 * P * P)[rows]
    conv = orc.mul_mat(pw.reshape(E, -1), orc.F32, 3 * P * P, E, np.ascontiguousarray(cols)).reshape(len(rows), E)
    pr = (rows // GRID % PG) * PG + (rows % GRID) % PG
    ref = ln_ref(orc, (conv + pos[pr]).astype(np.float32), lw, lb)
    assert np.abs(x.cpu().numpy()[rows] - ref).max() <= 1e-4
    ins, outs = {}, {}
    for i, blk in enumerate(blocks):
        if i in check:
            ins[i] = x.cpu().numpy()
        ctx.vit_block_forward(hp, blk, _p(x))
        if i in check:
            ctx.synchronize()
            outs[i] = x.cpu().numpy()
    ctx.synchronize()
    assert torch.equal(x, x_enc), "block-by-block run differs from mi355_vit_encode"
    for i in check:
        host, vec = hosts[i]
        g = int(i in GLOBAL_BLOCKS)
        _check_vit_block(orc, t, ins[i], outs[i], host, vec, g, fg if g else fw, 90 + i, f"encoder {tname} block {i}")


# ---------------------------------------------------------------- Hiera-tiny at 1024x1024
def _hiera_weights(mi, orc, t, info, seed):
    Cin, Cout = info.dim_in, info.dim_out
    shapes = {"qkv": (3 * Cout, Cin), "proj": (Cout, Cout), "fc1": (4 * Cout, Cout), "fc2": (Cout, 4 * Cout)}
    if Cin != Cout:
        shapes["dim_proj"] = (Cout, Cin)
    host, keep = {}, []
    blk = mi.HieraBlock()
    for i, (name, (N, K)) in enumerate(shapes.items()):
        q = orc.quantize_weights(t, orc.normal(N * K, seed, 30 + i, std=0.05).reshape(N, K))
        host[name] = (q, N, K)
        d = dev(q.view(np.uint8))
        keep.append(d)
        setattr(blk, name + "_w", mi.from_torch(d, t, [K, N]))
    vec = {}
    for i, (name, n, s, m) in enumerate([("norm1_w", Cin, 0.2, 1.0), ("norm1_b", Cin, 0.1, 0.0),
                                          ("qkv_b", 3 * Cout, 0.05, 0.0), ("proj_b", Cout, 0.05, 0.0),
                                          ("norm2_w", Cout, 0.2, 1.0), ("norm2_b", Cout, 0.1, 0.0),
                                          ("fc1_b", 4 * Cout, 0.05, 0.0), ("fc2_b", Cout, 0.05, 0.0),
                                          ("dim_proj_b", Cout, 0.05, 0.0)]):
        vec[name] = orc.normal(n, seed, 50 + i) * np.float32(s) + np.float32(m)
        d = dev(vec[name])
        keep.append(d)
        setattr(blk, name, d.data_ptr())
    return blk, host, vec, keep


def _check_hiera_block(orc, t, info, x_in, got, host, vec, S, what, seed):
    qsel = None
    if info.window_size == 0 and not info.q_stride and info.dim_in == info.dim_out:
        rng = np.random.default_rng(seed)
        qsel = np.sort(np.concatenate([[0, S * S - 1], rng.choice(np.arange(1, S * S - 1), 510, replace=False)]))
    rows, ref16 = hiera_block_ref(orc, t, x_in, info, host, vec, S, True, qsel=qsel)
    _, ref32 = hiera_block_ref(orc, t, x_in, info, host, vec, S, False, qsel=qsel)
    assert np.isfinite(got).all(), what
    return block_bars(got[rows], ref16, ref32, what)


@pytest.mark.parametrize("tname", ["f16", "q4_0"])
@pytest.mark.parametrize("idx,S", [(0, 256), (1, 256), (5, 64)])
def test_hiera_block_full(mi, ctx, orc, tname, idx, S):
    t = orc.NAME_TYPE[tname]
    hp = mi.hiera_tiny(1024)
    info = mi.hiera_block_info(hp, idx)
    blk, host, vec, _keep = _hiera_weights(mi, orc, t, info, seed=200 + idx)
    x0 = orc.normal(S * S * info.dim_in, 201, idx).reshape(S * S, info.dim_in)
    S2 = S // 2 if info.q_stride else S
    out = torch.full((S2 * S2, info.dim_out), float("nan"), dtype=torch.float32, device="cuda")
    print(f"hiera block {idx} {tname} S={S}", flush=True)
    ctx.hiera_block_forward(hp, idx, blk, _p(dev(x0)), S, _p(out))
    ctx.synchronize()
    _check_hiera_block(orc, t, info, x0, out.cpu().numpy(), host, vec, S, f"hiera block {idx} {tname}", 202 + idx)


@pytest.mark.parametrize("tname", ["f16", "q4_0"])
def test_hiera_encoder_stage_isolation(mi, ctx, orc, tname):
    """mi355_hiera_encode at 1024x1024: the patch embedding against the oracle,
    the blocks run one by one reproduce every stage output bit for bit, and
    every block's output against the oracle on that block's GPU input."""
    t = orc.NAME_TYPE[tname]
    hp = mi.hiera_tiny(1024)
    E0, S0 = 96, 256
    img = orc.uniform(3 * 1024 * 1024, 210, 1).reshape(3, 1024, 1024)
    pw = orc.normal(E0 * 147, 210, 2, std=0.05).reshape(E0, 3, 7, 7)
    pb = orc.normal(E0, 210, 3) * np.float32(0.05)
    pe = (orc.normal(S0 * S0 * E0, 210, 4) * np.float32(0.02)).reshape(S0 * S0, E0)
    infos, blocks, hosts, keep = [], [], [], []
    for i in range(12):
        info = mi.hiera_block_info(hp, i)
        blk, host, vec, k = _hiera_weights(mi, orc, t, info, seed=220 + i)
        infos.append(info)
        blocks.append(blk)
        hosts.append((host, vec))
        keep.append(k)
    dims = [(256, 96), (128, 192), (64, 384), (32, 768)]
    stage_out = [torch.full((s * s, c), float("nan"), dtype=torch.float32, device="cuda") for s, c in dims]
    imgd, pwd, pbd, ped = dev(img), dev(pw), dev(pb), dev(pe)
    print(f"hiera encoder {tname} at 1024x1024", flush=True)
    ctx.hiera_encode(hp, _p(imgd), mi.from_torch(pwd, mi.F32, [7, 7, 3, E0]), _p(pbd), _p(ped), blocks,
                     [o.data_ptr() for o in stage_out])
    ctx.synchronize()
    # patch embedding (ggml_conv_2d 7x7 / stride 4 / pad 3 + bias + pos_embed): block 0 on the GPU applied
    # to the oracle's embedding gives the stage-0 output up to the F32 GEMM's rounding (which may flip an
    # activation-quantization rounding inside block 0)
    pad = np.pad(img, ((0, 0), (3, 3), (3, 3)))
    win = np.lib.stride_tricks.sliding_window_view(pad, (7, 7), axis=(1, 2))[:, ::4, ::4]  # [3][S0][S0][7][7]
    cols = np.ascontiguousarray(win.transpose(1, 2, 0, 3, 4).reshape(S0 * S0, 147))
    conv = orc.mul_mat(pw.reshape(E0, -1), orc.F32, 147, E0, cols).reshape(S0 * S0, E0)
    x_emb = ((conv + pb).astype(np.float32) + pe).astype(np.float32)
    y0 = torch.full((S0 * S0, E0), float("nan"), dtype=torch.float32, device="cuda")
    ctx.hiera_block_forward(hp, 0, blocks[0], _p(dev(x_emb)), S0, _p(y0))
    ctx.synchronize()
    smax, srms = _check_hiera_block(orc, t, infos[0], x_emb, y0.cpu().numpy(), *hosts[0], S0,
                                    f"hiera encoder {tname} block 0", 230)
    # the two embeddings differ in the F32 GEMM's last bits: the stage-0 outputs may differ by the same
    # flipped roundings the oracle runs show, and no more
    de = np.abs(stage_out[0].cpu().numpy() - y0.cpu().numpy())
    print(f"stage 0 from the GPU vs the oracle embedding: max {de.max():.2e} rms {np.sqrt((de ** 2).mean()):.2e}")
    assert de.max() <= max(1e-2, 1.5 * smax) and np.sqrt((de ** 2).mean()) <= max(5e-4, 1.25 * srms)
    # blocks 1..11 from the encoder's stage-0 output, one at a time: every stage output bit for bit, and
    # every block against the oracle on its own GPU input
    x, S = stage_out[0], S0
    for i in range(1, 12):
        info = infos[i]
        S2 = S // 2 if info.q_stride else S
        y = torch.full((S2 * S2, info.dim_out), float("nan"), dtype=torch.float32, device="cuda")
        ctx.hiera_block_forward(hp, i, blocks[i], _p(x), S, _p(y))
        ctx.synchronize()
        _check_hiera_block(orc, t, info, x.cpu().numpy(), y.cpu().numpy(), *hosts[i], S,
                           f"hiera encoder {tname} block {i}", 230 + i)
        if i == 11 or infos[i + 1].stage != info.stage:
            assert torch.equal(stage_out[info.stage], y), \
                f"stage {info.stage}: block-by-block run differs from mi355_hiera_encode"
        x, S = y, S2
