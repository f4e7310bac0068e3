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
        quantized = t in (orc.Q8_0, orc.Q4_0, orc.Q4_1)
        assert blocks[0].fc1_w.layout == (mi.LAYOUT_INT8 if quantized else mi.LAYOUT_GGML)  # prepared at load
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


def test_hiera_from_file(mi, ctx, orc, tmp_path):
    """A SAM2 Hiera-tiny file at 128x128 (Q4_0): the loader derives the
    hyperparameters of sam2_load_hparams and builds the pos_embed table on the
    GPU; every stage output of the encoder run from the file's tables equals,
    bit for bit, the encoder fed the same bytes uploaded by hand with the
    oracle's sam2_compute_pos_embed table (so the loader's table is that table)."""
    t = orc.Q4_0
    hpw = mi.hiera_tiny(128)
    E, S0 = 96, 32
    rng = np.random.default_rng(17)
    f32 = lambda shape, s=0.05: (rng.standard_normal(shape) * s).astype(np.float32)
    ts = [("hiera.patch_embed.weight", orc.F32, (7, 7, 3, E), f32((E, 3, 7, 7))),
          ("hiera.patch_embed.bias", orc.F32, (E,), f32(E)),
          ("hiera.pos_embed", orc.F32, (7, 7, E, 1), f32((E, 7, 7), 0.1)),
          ("hiera.pos_embed_window", orc.F32, (8, 8, E, 1), f32((E, 8, 8), 0.1))]
    infos = [mi.hiera_block_info(hpw, i) for i in range(12)]
    for i, info in enumerate(infos):
        din, dout = info.dim_in, info.dim_out
        pre = f"hiera.blocks.{i}"
        mats = [(".attn.qkv.weight", din, 3 * dout), (".attn.proj.weight", dout, dout),
                (".mlp.fc1.weight", dout, 4 * dout), (".mlp.fc2.weight", 4 * dout, dout)]
        if din != dout:
            mats.append((".proj.weight", din, dout))
        for sfx, K, N in mats:
            ts.append((pre + sfx, t, (K, N), orc.quantize_weights(t, f32((N, K)))))
        vecs = [(".norm1.weight", din), (".norm1.bias", din), (".attn.qkv.bias", 3 * dout), (".attn.proj.bias", dout),
                (".norm2.weight", dout), (".norm2.bias", dout), (".mlp.fc1.bias", 4 * dout), (".mlp.fc2.bias", dout)]
        if din != dout:
            vecs.append((".proj.bias", dout))
        for sfx, n in vecs:
            ts.append((pre + sfx, orc.F32, (n,), f32(n, 0.2) + (np.float32(1) if "norm" in sfx and "weight" in sfx else 0)))
    rest = [E, 1, 4, 1, 2, 7, 2, 3, 5, 7, 9, 0, 0, 0, 0, 0, 3, 8, 4, 14, 7, 7, 7, 1] + [300 + i for i in range(31)]
    p = tmp_path / "hiera.ggml"
    W.write(p, W.MAGIC_SAM2, 1, 2, W.sam2_hparams(img=128, backbone=1, rest=rest), ts)
    f = mi.ModelFile(str(p))
    w, hp, blocks, n, pw, pb, pos = ctx.hiera_weights_load(f)
    try:
        assert n == 12 and (hp.img_size, hp.embed_dim, hp.num_heads, hp.q_pool) == (128, 96, 1, 3)
        assert list(hp.stages) == [1, 2, 7, 2] and list(hp.window_spec) == [8, 4, 14, 7]
        assert hp.n_global == 3 and list(hp.global_idx)[:3] == [5, 7, 9]
        by = {name: (tt, ne, data) for name, tt, ne, data in ts}
        pe_ref = orc.sam2_pos_embed(by["hiera.pos_embed"][2], by["hiera.pos_embed_window"][2], S0, S0)
        img = torch.from_numpy(orc.uniform(3 * 128 * 128, 9, 1).reshape(3, 128, 128)).cuda()
        dims = [(32, 96), (16, 192), (8, 384), (4, 768)]
        outs_f = [torch.full((s * s, c), float("nan"), dtype=torch.float32, device="cuda") for s, c in dims]
        ctx.hiera_encode(hp, C.c_void_p(img.data_ptr()), pw, C.c_void_p(pb), C.c_void_p(pos),
                         [blocks[i] for i in range(n)], [o.data_ptr() for o in outs_f])
        ctx.synchronize()
        # by hand: the same bytes, the oracle's pos_embed table
        keep = []

        def up(name):
            d = dev(np.ascontiguousarray(by[name][2]).view(np.uint8))
            keep.append(d)
            return d

        hb = []
        for i, info in enumerate(infos):
            pre = f"hiera.blocks.{i}"
            b = mi.HieraBlock()
            for fld, sfx in (("qkv_w", ".attn.qkv.weight"), ("proj_w", ".attn.proj.weight"),
                             ("fc1_w", ".mlp.fc1.weight"), ("fc2_w", ".mlp.fc2.weight"), ("dim_proj_w", ".proj.weight")):
                if pre + sfx in by:
                    tt, ne, _ = by[pre + sfx]
                    setattr(b, fld, mi.from_torch(up(pre + sfx), tt, list(ne)))
            for fld, sfx in (("norm1_w", ".norm1.weight"), ("norm1_b", ".norm1.bias"), ("qkv_b", ".attn.qkv.bias"),
                             ("proj_b", ".attn.proj.bias"), ("norm2_w", ".norm2.weight"), ("norm2_b", ".norm2.bias"),
                             ("fc1_b", ".mlp.fc1.bias"), ("fc2_b", ".mlp.fc2.bias"), ("dim_proj_b", ".proj.bias")):
                if pre + sfx in by:
                    setattr(b, fld, up(pre + sfx).data_ptr())
            hb.append(b)
        ped = dev(pe_ref)
        outs_h = [torch.full((s * s, c), float("nan"), dtype=torch.float32, device="cuda") for s, c in dims]
        ctx.hiera_encode(hpw, C.c_void_p(img.data_ptr()), mi.from_torch(up("hiera.patch_embed.weight"), orc.F32,
                                                                         [7, 7, 3, E]),
                         C.c_void_p(up("hiera.patch_embed.bias").data_ptr()), C.c_void_p(ped.data_ptr()), hb,
                         [o.data_ptr() for o in outs_h])
        ctx.synchronize()
        for a, b in zip(outs_f, outs_h):
            assert torch.isfinite(a).all()
            assert torch.equal(a, b)
    finally:
        ctx.hiera_weights_free(w)
