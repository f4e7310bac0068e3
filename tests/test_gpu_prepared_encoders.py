"""Encoders on prepared weights (mi355_weight_prepare): the fused producer
passes (LN, bias + GELU, the attention output) write the int8 kernel's
operand (one-byte quants, split scale dwords, Q8_1 sums for Q4_1) and every
quantized linear runs on the int8 kernel.  Bar: the block output is
bit-identical to the same block on the weights in the ggml layout (the fp16
kernels), fused and unfused, at the reduced test shapes and at the real SAM3
ViT width (E=1024, 72x72 tokens, 16 heads, MLP 4736); both are pinned to the
oracle by the encoder tests."""
import numpy as np
import pytest
import torch

import test_gpu_fullsize as full
import test_gpu_hiera as th
import test_gpu_vit as tv
from gpu_helpers import dev

pytestmark = pytest.mark.gpu


def _prepare(mi, ctx, wt, keep):
    n = mi.weight_prepared_nbytes(wt)
    buf = torch.full((n + 256,), 0xCD, dtype=torch.uint8, device="cuda")
    keep.append(buf)
    return ctx.weight_prepare(wt, buf.data_ptr() + (-buf.data_ptr()) % 256, n)


def _prepared_copy(mi, ctx, blk, cls, names, keep):
    """A copy of the block struct with every quantized weight prepared."""
    out = cls()
    for f, _ in cls._fields_:
        setattr(out, f, getattr(blk, f))
    for name in names:
        w = getattr(blk, name + "_w")
        if w.data and w.type in (2, 3, 8):
            setattr(out, name + "_w", _prepare(mi, ctx, w, keep))
    ctx.synchronize()
    return out


def _vit_run(ctx, hp, blk, x0, fuse=True):
    ctx.set_fusion(fuse)
    try:
        x = dev(x0)
        ctx.vit_block_forward(hp, blk, tv._p(x))
        ctx.synchronize()
    finally:
        ctx.set_fusion(True)
    return x


@pytest.mark.parametrize("is_global", [0, 1])
@pytest.mark.parametrize("tname", ["q8_0", "q4_0", "q4_1"])
def test_vit_block_prepared_bit_identical(mi, ctx, orc, is_global, tname):
    t = orc.NAME_TYPE[tname]
    E, NH, MLP, grid, ws = 256, 4, 1024, 48, 24
    HD = E // NH
    host, devs, vec = tv._block_weights(mi, orc, t, E, MLP, seed=27 + is_global)
    freqs = tv.axial_cis(orc, HD, grid, ws / grid) if is_global else tv.axial_cis(orc, HD, ws, 1.0)
    fd = dev(freqs)
    vd = {k: dev(v) for k, v in vec.items()}
    blk = mi.VitBlock()
    for name in ("qkv", "proj", "fc1", "fc2"):
        _, N, K = host[name]
        setattr(blk, name + "_w", mi.from_torch(devs[name], t, [K, N]))
    for k, v in vd.items():
        setattr(blk, k, v.data_ptr())
    blk.freqs_cis = fd.data_ptr()
    blk.is_global = is_global
    keep = []
    pblk = _prepared_copy(mi, ctx, blk, mi.VitBlock, ("qkv", "proj", "fc1", "fc2"), keep)
    hp = tv._hp(mi, E, NH, MLP, ws, grid)
    x0 = orc.normal(grid * grid * E, 29, 1).reshape(grid * grid, E)
    ref = _vit_run(ctx, hp, blk, x0)
    got = _vit_run(ctx, hp, pblk, x0)
    got_unfused = _vit_run(ctx, hp, pblk, x0, fuse=False)
    assert torch.isfinite(ref).all()
    assert torch.equal(got, ref), f"max diff {(got - ref).abs().max().item():.3e}"
    assert torch.equal(got_unfused, ref), f"max diff {(got_unfused - ref).abs().max().item():.3e}"


@pytest.mark.parametrize("is_global", [0, 1])
@pytest.mark.parametrize("tname", ["q8_0", "q4_0"])
def test_vit_block_full_prepared_bit_identical(mi, ctx, orc, is_global, tname):
    t = orc.NAME_TYPE[tname]
    fd = dev(full._freqs(orc, is_global))
    blk, _host, _vec, keep = full._vit_block_weights(mi, orc, t, 90 + is_global, is_global, fd)
    pkeep = []
    pblk = _prepared_copy(mi, ctx, blk, mi.VitBlock, ("qkv", "proj", "fc1", "fc2"), pkeep)
    x0 = orc.normal(full.GRID * full.GRID * full.E, 91, 1).reshape(full.GRID * full.GRID, full.E)
    print(f"vit block E={full.E} grid={full.GRID} {tname} global={is_global}: prepared vs ggml layout", flush=True)
    ref = _vit_run(ctx, full._hp(mi), blk, x0)
    got = _vit_run(ctx, full._hp(mi), pblk, x0)
    assert torch.isfinite(ref).all()
    assert torch.equal(got, ref), f"max diff {(got - ref).abs().max().item():.3e}"


@pytest.mark.parametrize("tname", ["q8_0", "q4_0"])
def test_vit_encode_prepared_layernorm_handoff(mi, ctx, orc, tname):
    """On prepared weights mi355_vit_encode gives each block's fc2 the next block's LN1 (at
    E = 1024 in one pass with fc2's K-split reduction, into the window or image order the
    next block needs): the encoder equals the prefix plus mi355_vit_block_forward block by
    block, and the encoder on the ggml-layout weights, bit for bit.  Four blocks at the real
    SAM3 width: windowed, global, windowed, windowed."""
    t = orc.NAME_TYPE[tname]
    S = full.GRID * full.P
    img = orc.uniform(3 * S * S, 95, 1).reshape(3, S, S)
    pw = orc.normal(full.E * 3 * full.P * full.P, 95, 2, std=0.02).reshape(full.E, 3, full.P, full.P)
    pos = orc.normal(full.PG * full.PG * full.E, 95, 3).reshape(full.PG * full.PG, full.E)
    lw = orc.normal(full.E, 95, 4) * np.float32(0.2) + np.float32(1.0)
    lb = orc.normal(full.E, 95, 5) * np.float32(0.1)
    fw, fg = dev(full._freqs(orc, 0)), dev(full._freqs(orc, 1))
    raw, prep, keep = [], [], []
    for i, g in enumerate((0, 1, 0, 0)):
        blk, _host, _vec, k = full._vit_block_weights(mi, orc, t, 130 + i, g, fg if g else fw)
        keep.append(k)
        raw.append(blk)
        prep.append(_prepared_copy(mi, ctx, blk, mi.VitBlock, ("qkv", "proj", "fc1", "fc2"), keep))
    hp = full._hp(mi)
    imgd, pwd, posd, lwd, lbd = dev(img), dev(pw), dev(pos), dev(lw), dev(lb)
    patch = mi.from_torch(pwd, mi.F32, [full.P, full.P, 3, full.E])
    print(f"vit encode {tname}: 4 blocks at E={full.E}, prepared and ggml layout", flush=True)
    outs = {}
    for name, blocks in (("prepared", prep), ("ggml", raw)):
        x = torch.empty((full.GRID * full.GRID, full.E), dtype=torch.float32, device="cuda")
        ctx.vit_encode(hp, tv._p(imgd), patch, tv._p(posd), tv._p(lwd), tv._p(lbd), blocks, tv._p(x))
        outs[name] = x
    x = torch.empty_like(outs["prepared"])
    ctx.vit_prefix(hp, tv._p(imgd), patch, tv._p(posd), tv._p(lwd), tv._p(lbd), tv._p(x))
    for blk in prep:
        ctx.vit_block_forward(hp, blk, tv._p(x))
    ctx.synchronize()
    assert torch.isfinite(x).all()
    assert torch.equal(outs["prepared"], x), f"max diff {(outs['prepared'] - x).abs().max().item():.3e}"
    assert torch.equal(outs["ggml"], x), f"max diff {(outs['ggml'] - x).abs().max().item():.3e}"


@pytest.mark.parametrize("tname", ["q8_0", "q4_0", "q4_1"])
@pytest.mark.parametrize("idx,S", th.CASES)
def test_hiera_block_prepared_bit_identical(mi, ctx, orc, tname, idx, S):
    t = orc.NAME_TYPE[tname]
    hp = mi.hiera_tiny(128)
    info = mi.hiera_block_info(hp, idx)
    host, devs, vec = th._weights(mi, orc, t, info, seed=idx + 31)
    blk, _keep = th._block_dev(mi, t, host, devs, vec)
    keep = []
    pblk = _prepared_copy(mi, ctx, blk, mi.HieraBlock, ("qkv", "proj", "fc1", "fc2", "dim_proj"), keep)
    x0 = orc.normal(S * S * info.dim_in, idx, 63).reshape(S * S, info.dim_in)
    S2 = S // 2 if info.q_stride else S
    xd = dev(x0)
    outs = []
    for b in (blk, pblk):
        out = torch.full((S2 * S2, info.dim_out), float("nan"), dtype=torch.float32, device="cuda")
        ctx.hiera_block_forward(hp, idx, b, th._p(xd), S, th._p(out))
        ctx.synchronize()
        outs.append(out)
    assert torch.isfinite(outs[0]).all()
    assert torch.equal(outs[1], outs[0]), f"max diff {(outs[1] - outs[0]).abs().max().item():.3e}"


@pytest.mark.parametrize("tname", ["q8_0", "q4_0"])
@pytest.mark.parametrize("idx", [0, 1])
def test_hiera_block_prepared_65536_tokens_bit_identical(mi, ctx, orc, tname, idx):
    """Hiera-tiny blocks 0 and 1 at S = 256 (65536 tokens, K = 96 projections): on prepared
    weights the stage-1 qkv (qkv epilogue), proj (residual epilogue), fc1 and dim_proj run on
    the int8 kernel at 64-row tiles; on ggml-layout weights the K = 96 stores take the fp16
    skinny kernel.  Bar: both blocks give the same bits."""
    t = orc.NAME_TYPE[tname]
    S = 256
    hp = mi.hiera_tiny(1024)
    info = mi.hiera_block_info(hp, idx)
    host, devs, vec = th._weights(mi, orc, t, info, seed=idx + 41)
    blk, _keep = th._block_dev(mi, t, host, devs, vec)
    keep = []
    pblk = _prepared_copy(mi, ctx, blk, mi.HieraBlock, ("qkv", "proj", "fc1", "fc2", "dim_proj"), keep)
    x0 = orc.normal(S * S * info.dim_in, idx, 67).reshape(S * S, info.dim_in)
    S2 = S // 2 if info.q_stride else S
    xd = dev(x0)
    print(f"hiera block {idx} S={S} {tname}: prepared vs ggml layout", flush=True)
    outs = []
    for b in (pblk, blk):
        out = torch.full((S2 * S2, info.dim_out), float("nan"), dtype=torch.float32, device="cuda")
        ctx.hiera_block_forward(hp, idx, b, th._p(xd), S, th._p(out))
        ctx.synchronize()
        outs.append(out)
    assert torch.isfinite(outs[0]).all()
    assert torch.equal(outs[0], outs[1]), f"max diff {(outs[0] - outs[1]).abs().max().item():.3e}"
