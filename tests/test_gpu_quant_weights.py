"""GPU weight quantize and the model-file quantizer.

mi355_quantize_weights (ggml_quantize_chunk with the _ref row quantizers,
examples/quantize.cpp:244-245) is bit-exact with the oracle's
quantize_row_{q8_0,q4_0,q4_1}_ref on random rows, the known-answer blocks,
first-extreme ties and signed zeros, from F32 and F16 sources.

mi355_model_quantize (sam3_quantize_model, examples/quantize.cpp:20-331)
writes, byte for byte, the file that the reference's rule describes: header
ftype = qtype, hyperparameters and kept tensors copied, quantized tensors as
the oracle quantizes them, 32-byte record padding, the tail copied; a SAM3
ViT file quantized from F32 equals the file written with oracle-quantized
weights from the same draws."""
import ctypes as C
import json
import os

import numpy as np
import pytest
import torch

import model_file_writer as W
from gpu_helpers import dev

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def gpu_quantize_weights(mi, ctx, t, x, src_type=None, pitch=None):
    """x [rows, K] float32 (or float16 when src_type is F16); pitch in elements."""
    rows, k = x.shape
    src_type = mi.F32 if src_type is None else src_type
    esz = 4 if src_type == mi.F32 else 2
    pitch = k if pitch is None else pitch
    buf = np.zeros((rows, pitch), dtype=x.dtype)
    buf[:, :k] = x
    xd = dev(buf.view(np.uint8))
    rs = mi.row_size(t, k)
    out = torch.zeros(rows * rs + 16, dtype=torch.uint8, device="cuda")
    src = mi.from_torch(xd, src_type, [k, rows], [esz, pitch * esz, pitch * esz * rows, pitch * esz * rows])
    ctx.quantize_weights(t, src, out.data_ptr())
    ctx.synchronize()
    return out[: rows * rs].cpu().numpy().reshape(rows, rs)


def special_blocks(orc):
    with open(os.path.join(HERE, "golden", "quant_kat.json")) as f:
        kat = json.load(f)
    rows = [np.array(c["x"], np.float32) for key in ("q8_act", "q4_0", "q4_1") for c in kat[key]]
    z = np.zeros(32, np.float32)
    for pair in ((2.0, -2.0), (-2.0, 2.0), (-0.0, 0.0), (0.0, -0.0)):
        b = z.copy()
        b[5], b[21] = pair
        b[9] = 1.0
        rows.append(b)
    tiny = np.full(32, 1e-30, np.float32)
    tiny[3] = -2e-30
    rows += [z, tiny, orc.normal(32, 9, 9) * np.float32(1e4), np.full(32, -3.25, np.float32)]
    return np.concatenate(rows)


@pytest.mark.parametrize("tname", ["q8_0", "q4_0", "q4_1"])
@pytest.mark.parametrize("src", ["f32", "f16"])
def test_quantize_weights_bit_exact(mi, ctx, orc, tname, src):
    t = orc.NAME_TYPE[tname]
    K = 1024
    x = orc.normal(300 * K, seed=2, stream=7, std=0.02).reshape(300, K)
    sp = special_blocks(orc)
    x[0, : sp.size] = sp
    if src == "f16":
        x16 = x.astype(np.float16)
        out = gpu_quantize_weights(mi, ctx, t, x16, mi.F16)
        ref = orc.quantize_weights(t, x16.astype(np.float32))
    else:
        out = gpu_quantize_weights(mi, ctx, t, x)
        ref = orc.quantize_weights(t, x)
    bad = np.nonzero((out != ref).any(axis=1))[0]
    assert bad.size == 0, f"rows differ: {bad[:8]}"


def test_quantize_weights_ties_hand_derived(mi, ctx):
    """The first of equal extremes wins (hand-derived bytes, as in the oracle's
    own test): Q4_0 [2, -2, 0..] -> d = -0.25, [-2, 2, 0..] -> d = +0.25;
    Q4_1 [-0.0, 0.0, 1, 0..] -> m = -0.0, [0.0, -0.0, 1, ..] -> m = +0.0."""
    z = np.zeros(32, np.float32)
    a, b = z.copy(), z.copy()
    a[0], a[1] = 2.0, -2.0
    b[0], b[1] = -2.0, 2.0
    q = gpu_quantize_weights(mi, ctx, mi.Q4_0, np.stack([a, b]))
    assert q[:, 0:2].copy().view(np.uint16)[:, 0].tolist() == [0xB400, 0x3400]
    assert q[0, 2:18].tolist() == q[1, 2:18].tolist() == [0x80, 0x8F] + [0x88] * 14
    c0, c1 = z.copy(), z.copy()
    c0[0], c0[1], c0[2] = -0.0, 0.0, 1.0
    c1[0], c1[1], c1[2] = 0.0, -0.0, 1.0
    q = gpu_quantize_weights(mi, ctx, mi.Q4_1, np.stack([c0, c1]))
    assert q[:, 0:4].copy().view(np.uint16).tolist() == [[0x2C44, 0x8000], [0x2C44, 0x0000]]
    assert q[0, 4:20].tolist() == q[1, 4:20].tolist() == [0, 0, 15] + [0] * 13


@pytest.mark.parametrize("tname", ["q8_0", "q4_0", "q4_1"])
def test_quantize_weights_row_pitch(mi, ctx, orc, tname):
    """Rows with a pitch beyond ne0 (a view into a wider buffer): same bytes."""
    t = orc.NAME_TYPE[tname]
    x = orc.normal(37 * 96, seed=3, stream=1).reshape(37, 96)
    out = gpu_quantize_weights(mi, ctx, t, x, pitch=131)
    assert np.array_equal(out, orc.quantize_weights(t, x))


# ---------------------------------------------------------------- file tool

def _tensors(orc, rng):
    """(name, type, ne, data, quantized?) covering the reference's rule."""
    f32 = lambda *shape: (rng.standard_normal(shape) * 0.05).astype(np.float32)
    q8 = orc.quantize_weights(orc.Q8_0, f32(4, 64))
    return [
        ("vit.blocks.0.attn.qkv.weight", orc.F32, (64, 96), f32(96, 64), True),
        ("vit.blocks.0.mlp.lin1.weight", orc.F16, (64, 128), f32(128, 64).astype(np.float16), True),
        ("vit.blocks.0.norm1.weight", orc.F32, (64,), f32(64), False),           # 1-D
        ("vit.pos_embed", orc.F32, (64, 4, 4, 1), f32(1, 4, 4, 64), False),      # name: pos_embed
        ("sam_dec.iou_token.weight", orc.F32, (64, 1), f32(1, 64), False),       # name: iou_token
        ("ddec.bbox_embed.layers.0.weight", orc.F32, (64, 64), f32(64, 64), True),  # "embed" alone does not keep
        ("neck.conv.weight", orc.F16, (32, 3, 3, 8), f32(8, 3, 3, 32).astype(np.float16), True),  # 4-D
        ("neck.conv3.weight", orc.F32, (3, 3, 64, 8), f32(8, 64, 3, 3), False),   # ne0 = 3
        ("odd.weight", orc.F32, (48, 8), f32(8, 48), False),                     # ne0 % 32 != 0
        ("pre.q8.weight", orc.Q8_0, (64, 4), q8, False),                         # already quantized
        ("x.freqs_cis", orc.F32, (64, 2), f32(2, 64), False),                    # name: freqs_cis
    ]


def _expected(orc, ts, qtype):
    out = []
    for name, t, ne, data, quant in ts:
        if quant:
            x = np.asarray(data).astype(np.float32).reshape(-1, ne[0])
            out.append((name, qtype, ne, orc.quantize_weights(qtype, x)))
        else:
            out.append((name, t, ne, data))
    return out


@pytest.mark.parametrize("kind", ["sam3", "sam2", "edgetam"])
@pytest.mark.parametrize("qname", ["q8_0", "q4_0", "q4_1"])
def test_model_quantize_bytes(mi, ctx, orc, tmp_path, kind, qname):
    qtype = orc.NAME_TYPE[qname]
    ts = _tensors(orc, np.random.default_rng(4))
    if kind == "sam3":
        magic, ver, hp = W.MAGIC_SAM3, 3, W.sam3_hparams(global_idx=(2, 5, 8, 11))
    elif kind == "sam2":
        magic, ver, hp = W.MAGIC_SAM2, 1, W.sam2_hparams()
    else:  # backbone_type 2 carries 19 more hyperparameters
        magic, ver, hp = W.MAGIC_SAM2, 1, W.sam2_hparams(backbone=2, rest=[300 + i for i in range(55 + 19)])
    tail = b"tokenizer\x00" + bytes(range(200))
    src, dst, want = tmp_path / "in.ggml", tmp_path / "out.ggml", tmp_path / "want.ggml"
    W.write(src, magic, ver, 1, hp, [t[:4] for t in ts], tail=tail)
    W.write(want, magic, ver, qtype, hp, _expected(orc, ts, qtype), tail=tail)
    st = ctx.model_quantize(src, dst, qtype)
    assert dst.read_bytes() == want.read_bytes()
    nq = sum(t[4] for t in ts)
    assert (st.n_quantized, st.n_total) == (nq, len(ts))
    assert st.size_org == sum(4 * int(np.prod(t[2])) for t in ts)
    assert st.size_new == sum(np.asarray(e[3]).nbytes for e in _expected(orc, ts, qtype))


@pytest.mark.parametrize("qname", ["q8_0", "q4_0"])
def test_model_quantize_vit_file(mi, ctx, orc, tmp_path, qname):
    """An F32 SAM3 ViT file quantized on the GPU is the file written directly
    with the oracle's quantized weights from the same draws, and it loads."""
    from test_gpu_model_file import _vit_file
    t = orc.NAME_TYPE[qname]
    f32, direct, out = tmp_path / "f32.ggml", tmp_path / "direct.ggml", tmp_path / "out.ggml"
    _vit_file(orc, f32, 0, orc.F32)
    _vit_file(orc, direct, t, t)
    ctx.model_quantize(f32, out, t)
    assert out.read_bytes() == direct.read_bytes()
    f = mi.ModelFile(str(out))
    w, hp, blocks, n, pw, pos, lw, lb = ctx.vit_weights_load(f)
    try:
        assert blocks[0].qkv_w.type == t and pw.type == orc.F32
    finally:
        ctx.vit_weights_free(w)


def test_model_quantize_errors(mi, ctx, orc, tmp_path):
    rng = np.random.default_rng(6)
    w = (rng.standard_normal((4, 64)) * 0.1).astype(np.float32)
    good = [("a.weight", orc.F32, (64, 4), w)]
    out = tmp_path / "o.ggml"

    def status(path, qtype=orc.Q8_0):
        with pytest.raises(mi.Mi355Error) as e:
            ctx.model_quantize(path, out, qtype)
        assert not out.exists()  # no half-written model is left behind
        return e.value.status

    p = tmp_path / "magic.ggml"
    W.write(p, 0x12345678, 3, 0, W.sam3_hparams(), good)
    assert status(p) == -4
    p = tmp_path / "version.ggml"
    W.write(p, W.MAGIC_SAM3, 2, 0, W.sam3_hparams(), good)
    assert status(p) == -3
    p = tmp_path / "type.ggml"
    W.write(p, W.MAGIC_SAM3, 3, 0, W.sam3_hparams(), good + [("q5.weight", 6, (64, 4), np.zeros(88, np.uint8))])
    assert status(p) == -3
    p = tmp_path / "short.ggml"
    W.write(p, W.MAGIC_SAM3, 3, 0, W.sam3_hparams(), good)
    p.write_bytes(p.read_bytes()[:-100])
    assert status(p) == -1
    p = tmp_path / "ok.ggml"
    W.write(p, W.MAGIC_SAM3, 3, 0, W.sam3_hparams(), good)
    assert status(p, orc.F16) == -3
    assert status(tmp_path / "missing.ggml") == -1
    big = 2**31 - 1                                  # element count past int64
    p = tmp_path / "huge.ggml"
    W.write(p, W.MAGIC_SAM3, 3, 0, W.sam3_hparams(), good + [("h.weight", orc.F32, (big, big, big), np.zeros(8, np.uint8))])
    assert status(p) == -3
    p = tmp_path / "long.ggml"                       # 2^61 bytes claimed in a tiny file
    W.write(p, W.MAGIC_SAM3, 3, 0, W.sam3_hparams(), good + [("l.weight", orc.F32, (2**30, 2**29), np.zeros(8, np.uint8))])
    assert status(p) == -1
