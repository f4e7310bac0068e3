"""Loading .ggml model files into device memory (sam3_load_tensors,
sam3.cpp:3095-3198) and running the SAM3 ViT from a file.

Bars: same-type loads are the file's bytes; F16->F32, F32->F16 (round to
nearest even) and Q8_0/Q4_0/Q4_1 -> F32 dequantization are bit-exact against
numpy / the oracle's dequantize; a ViT encoded from file weights equals, bit
for bit, the same encoder fed the same bytes uploaded by hand."""
import ctypes as C

import numpy as np
import pytest
import torch

import model_file_writer as W
from gpu_helpers import dev

pytestmark = pytest.mark.gpu


def _load(mi, ctx, f, i, t):
    nb = f.load_bytes(i, t)
    buf = torch.empty(nb, dtype=torch.uint8, device="cuda")
    ctx.model_file_load(f, i, t, buf.data_ptr(), nb)
    ctx.synchronize()
    return buf.cpu().numpy()


def test_load_and_convert(mi, ctx, orc, tmp_path):
    rng = np.random.default_rng(5)
    w = rng.standard_normal((40, 96)).astype(np.float32) * np.float32(0.1)
    f16 = (rng.standard_normal(333) * 3).astype(np.float16)
    f32 = (rng.standard_normal(257) * 100).astype(np.float32)
    ts = [("f16", orc.F16, (333,), f16), ("f32", orc.F32, (257,), f32)]
    for name, t in (("q8_0", orc.Q8_0), ("q4_0", orc.Q4_0), ("q4_1", orc.Q4_1)):
        ts.append((name, t, (96, 40), orc.quantize_weights(t, w)))
    p = tmp_path / "m.ggml"
    W.write(p, W.MAGIC_SAM3, 3, 8, W.sam3_hparams(), ts)
    f = mi.ModelFile(str(p))
    for i, (name, t, ne, data) in enumerate(ts):
        assert _load(mi, ctx, f, i, t).tobytes() == np.ascontiguousarray(data).tobytes(), name
    assert np.array_equal(_load(mi, ctx, f, 0, mi.F32).view(np.float32), f16.astype(np.float32))
    assert np.array_equal(_load(mi, ctx, f, 1, mi.F16).view(np.float16), f32.astype(np.float16))
    for i in (2, 3, 4):
        name, t, ne, data = ts[i]
        got = _load(mi, ctx, f, i, mi.F32).view(np.float32).reshape(40, 96)
        ref = orc.dequantize(t, data, 96)
        assert np.array_equal(got, ref), name


def _vit_file(orc, path, ftype, t, seed=3):
    E, NH, depth, img, P, ws = 256, 4, 2, 672, 14, 24
    MLP, G, HD = 1024, img // P, E // NH
    pg = G // 3
    rng = np.random.default_rng(seed)
    wt = lambda ne0: t if ne0 % (32 if t not in (orc.F32, orc.F16) else 1) == 0 else orc.F32

    def weight(name, ne0, ne1, std=0.02):
        x = rng.standard_normal((ne1, ne0)).astype(np.float32) * np.float32(std)
        tt = wt(ne0)
        data = orc.quantize_weights(tt, x) if tt != orc.F32 else x
        return (name, tt, (ne0, ne1), data)

    def vec(name, n, s=0.1, m=0.0):
        return (name, orc.F32, (n,), (rng.standard_normal(n) * s + m).astype(np.float32))

    ts = [("vit.patch_embed.proj.weight", wt(P), (P, P, 3, E),
           orc.quantize_weights(wt(P), rng.standard_normal((E * 3 * P, P)).astype(np.float32) * np.float32(0.02))
           if wt(P) != orc.F32 else rng.standard_normal((E, 3, P, P)).astype(np.float32) * np.float32(0.02)),
          ("vit.pos_embed", orc.F32, (E, pg, pg, 1), rng.standard_normal((pg * pg, E)).astype(np.float32)),
          vec("vit.ln_pre.weight", E, 0.2, 1.0), vec("vit.ln_pre.bias", E)]
    for i in range(depth):
        pre = f"vit.blocks.{i}"
        glob = i == 1
        n = G * G if glob else ws * ws
        ang = rng.uniform(0, 6.28, size=(n, HD // 2)).astype(np.float32)
        cis = np.stack([np.cos(ang), np.sin(ang)], axis=-1).astype(np.float32)
        ts += [vec(pre + ".norm1.weight", E, 0.2, 1.0), vec(pre + ".norm1.bias", E),
               weight(pre + ".attn.qkv.weight", E, 3 * E), vec(pre + ".attn.qkv.bias", 3 * E, 0.05),
               weight(pre + ".attn.proj.weight", E, E), vec(pre + ".attn.proj.bias", E, 0.05),
               vec(pre + ".norm2.weight", E, 0.2, 1.0), vec(pre + ".norm2.bias", E),
               weight(pre + ".mlp.lin1.weight", E, MLP), vec(pre + ".mlp.lin1.bias", MLP, 0.05),
               weight(pre + ".mlp.lin2.weight", MLP, E), vec(pre + ".mlp.lin2.bias", E, 0.05),
               (pre + ".attn.freqs_cis", orc.F32, (2, HD // 2, n), cis)]
    hp = W.sam3_hparams(img=img, patch=P, embed=E, depth=depth, heads=NH, mlp_x1000=4000, window=ws,
                        global_idx=(1,))
    W.write(path, W.MAGIC_SAM3, 3, ftype, hp, ts)
    return ts, dict(E=E, NH=NH, MLP=MLP, G=G, ws=ws, P=P, pg=pg, img=img)


@pytest.mark.parametrize("tname,ftype", [("q8_0", 8), ("q4_0", 2), ("f16", 1)])
def test_vit_from_file(mi, ctx, orc, tmp_path, tname, ftype):
    t = orc.NAME_TYPE[tname]
    p = tmp_path / "vit.ggml"
    ts, g = _vit_file(orc, p, ftype, t)
    f = mi.ModelFile(str(p))
    w, hp, blocks, n, pw, pos, lw, lb = ctx.vit_weights_load(f)
    try:
        assert (hp.embed_dim, hp.num_heads, hp.mlp_dim, hp.window_size, hp.grid, hp.patch_size, hp.pos_grid) == \
            (g["E"], g["NH"], g["MLP"], g["ws"], g["G"], g["P"], g["pg"])
        assert n == 2 and blocks[0].is_global == 0 and blocks[1].is_global == 1
        img = torch.from_numpy(orc.uniform(3 * g["img"] ** 2, 4, 1).reshape(3, g["img"], g["img"])).cuda()
        x_file = torch.empty((g["G"] ** 2, g["E"]), dtype=torch.float32, device="cuda")
        ctx.vit_encode(hp, C.c_void_p(img.data_ptr()), pw, C.c_void_p(pos), C.c_void_p(lw), C.c_void_p(lb),
                       [blocks[i] for i in range(n)], C.c_void_p(x_file.data_ptr()))
        ctx.synchronize()
        # the same bytes uploaded by hand into the block table the encoder takes
        by = {name: (tt, ne, data) for name, tt, ne, data in ts}
        keep = []

        def up(name):
            d = dev(np.ascontiguousarray(by[name][2]).view(np.uint8))
            keep.append(d)
            return d

        def ten(name):
            tt, ne, _ = by[name]
            return mi.from_torch(up(name), tt, list(ne) + [1] * (4 - len(ne)))

        hb = (mi.VitBlock * 2)()
        for i in range(2):
            pre = f"vit.blocks.{i}"
            hb[i].qkv_w, hb[i].proj_w = ten(pre + ".attn.qkv.weight"), ten(pre + ".attn.proj.weight")
            hb[i].fc1_w, hb[i].fc2_w = ten(pre + ".mlp.lin1.weight"), ten(pre + ".mlp.lin2.weight")
            for fld, nm in (("norm1_w", ".norm1.weight"), ("norm1_b", ".norm1.bias"), ("qkv_b", ".attn.qkv.bias"),
                            ("proj_b", ".attn.proj.bias"), ("norm2_w", ".norm2.weight"),
                            ("norm2_b", ".norm2.bias"), ("fc1_b", ".mlp.lin1.bias"), ("fc2_b", ".mlp.lin2.bias"),
                            ("freqs_cis", ".attn.freqs_cis")):
                setattr(hb[i], fld, up(pre + nm).data_ptr())
            hb[i].is_global = 1 if i == 1 else 0
        x_hand = torch.empty_like(x_file)
        ctx.vit_encode(hp, C.c_void_p(img.data_ptr()), ten("vit.patch_embed.proj.weight"),
                       C.c_void_p(up("vit.pos_embed").data_ptr()), C.c_void_p(up("vit.ln_pre.weight").data_ptr()),
                       C.c_void_p(up("vit.ln_pre.bias").data_ptr()), list(hb), C.c_void_p(x_hand.data_ptr()))
        ctx.synchronize()
        a, b = x_file.cpu().numpy(), x_hand.cpu().numpy()
        assert np.isfinite(a).all()
        assert np.array_equal(a, b)
    finally:
        ctx.vit_weights_free(w)
