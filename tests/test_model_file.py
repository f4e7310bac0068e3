"""The .ggml model-file reader (sam3_load_model / sam3_load_tensors,
sam3.cpp:3095-3348) on the host: header and hyperparameters of SAM3 and SAM2
files, the tensor index (types, ggml shapes, 32-byte aligned data offsets, data
sizes as ggml_row_size gives them), the conversions a load may apply, and the
rejections.  Files are written by tests/model_file_writer.py."""
import numpy as np
import pytest

import model_file_writer as W


def _tensors(orc):
    rng = np.random.default_rng(0)
    w = rng.standard_normal((8, 64)).astype(np.float32) * np.float32(0.05)
    return [
        ("a.f32", orc.F32, (5,), rng.standard_normal(5).astype(np.float32)),
        ("b.f16", orc.F16, (3, 7), rng.standard_normal(21).astype(np.float16)),
        ("c.q8_0", orc.Q8_0, (64, 8), orc.quantize_weights(orc.Q8_0, w)),
        ("d.q4_0", orc.Q4_0, (64, 8), orc.quantize_weights(orc.Q4_0, w)),
        ("e.q4_1", orc.Q4_1, (64, 4, 2), orc.quantize_weights(orc.Q4_1, w)),
        ("f.four_dims", orc.F32, (2, 3, 4, 5), np.arange(120, dtype=np.float32)),
    ]


def test_sam3_file_index(mi, orc, tmp_path):
    p = tmp_path / "m.ggml"
    hp = W.sam3_hparams()
    ts = _tensors(orc)
    W.write(p, W.MAGIC_SAM3, 3, 8, hp, ts, pad_byte=0x5A)
    f = mi.ModelFile(str(p))
    assert f.header() == (W.MAGIC_SAM3, 3, 8, len(ts))
    assert f.hparams() == hp
    raw = p.read_bytes()
    for i, (name, t, ne, data) in enumerate(ts):
        info = f.tensor(i)
        assert info["name"] == name and info["type"] == t and info["n_dims"] == len(ne)
        assert info["ne"] == list(ne) + [1] * (4 - len(ne))
        assert info["offset"] % 32 == 0
        nel = int(np.prod(ne))
        assert info["nbytes"] == (orc.row_size(t, ne[0]) * (nel // ne[0]))
        assert raw[info["offset"]:info["offset"] + info["nbytes"]] == np.ascontiguousarray(data).tobytes()
        assert f.find(name) == i
        assert f.load_bytes(i, t) == info["nbytes"]
        assert f.load_bytes(i, mi.F32) == nel * 4
    assert f.find("missing") == -1
    # conversions sam3_load_tensors applies: F16<->F32, quantized -> F32 only
    assert f.load_bytes(1, mi.F16) == 21 * 2 and f.load_bytes(0, mi.F16) == 5 * 2
    assert f.load_bytes(2, mi.F16) == 0 and f.load_bytes(2, mi.Q4_0) == 0
    f.close()


@pytest.mark.parametrize("n_global", [0, 1, 4, 6])
def test_sam3_global_list_length(mi, orc, tmp_path, n_global):
    """sam3_load_hparams reads min(n_global, 4) block indices."""
    p = tmp_path / "m.ggml"
    hp = W.sam3_hparams(global_idx=tuple(range(10, 10 + n_global)))
    hp[7] = n_global
    W.write(p, W.MAGIC_SAM3, 3, 1, hp, _tensors(orc)[:1])
    f = mi.ModelFile(str(p))
    assert len(f.hparams()) == 8 + min(n_global, 4) + 27
    assert f.tensor(0)["name"] == "a.f32"


def test_sam2_file(mi, orc, tmp_path):
    p = tmp_path / "m.ggml"
    hp = W.sam2_hparams()
    W.write(p, W.MAGIC_SAM2, 1, 2, hp, _tensors(orc)[2:4])
    f = mi.ModelFile(str(p))
    assert f.header() == (W.MAGIC_SAM2, 1, 2, 2)
    assert f.hparams() == hp and len(hp) == 57
    assert [f.tensor(i)["name"] for i in range(2)] == ["c.q8_0", "d.q4_0"]


def _expect_error(mi, path, code):
    with pytest.raises(mi.Mi355Error) as e:
        mi.ModelFile(str(path))
    assert e.value.status == code, e.value


def test_rejections(mi, orc, tmp_path):
    ts = _tensors(orc)
    p = tmp_path / "m.ggml"
    W.write(p, 0x12345678, 3, 8, W.sam3_hparams(), ts)
    _expect_error(mi, p, -4)                                        # unknown magic
    W.write(p, W.MAGIC_SAM3, 2, 8, W.sam3_hparams(), ts)
    _expect_error(mi, p, -3)                                        # SAM3 version
    W.write(p, W.MAGIC_SAM2, 2, 8, W.sam2_hparams(), ts)
    _expect_error(mi, p, -3)                                        # SAM2 version
    W.write(p, W.MAGIC_SAM3, 3, 6, W.sam3_hparams(), ts)
    _expect_error(mi, p, -3)                                        # ftype
    W.write(p, W.MAGIC_SAM2, 1, 8, W.sam2_hparams(backbone=2), ts)
    _expect_error(mi, p, -3)                                        # EdgeTAM backbone
    W.write(p, W.MAGIC_SAM3, 3, 8, W.sam3_hparams(), ts + [ts[0]])
    _expect_error(mi, p, -4)                                        # duplicate name
    W.write(p, W.MAGIC_SAM3, 3, 8, W.sam3_hparams(), [("bad", 6, (32,), np.zeros(4, np.uint8))])
    _expect_error(mi, p, -3)                                        # unsupported tensor type
    W.write(p, W.MAGIC_SAM3, 3, 8, W.sam3_hparams(), [("odd", orc.Q8_0, (48,), np.zeros(51, np.uint8))])
    _expect_error(mi, p, -3)                                        # rows not whole blocks
    W.write(p, W.MAGIC_SAM3, 3, 8, W.sam3_hparams(), ts)
    data = p.read_bytes()
    p.write_bytes(data[:-10])
    _expect_error(mi, p, -1)                                        # truncated data
    _expect_error(mi, tmp_path / "absent.ggml", -1)
    big = 2**31 - 1                                                 # element count past int64
    W.write(p, W.MAGIC_SAM3, 3, 8, W.sam3_hparams(), [("huge", orc.F32, (big, big, big), np.zeros(8, np.uint8))])
    _expect_error(mi, p, -3)
    W.write(p, W.MAGIC_SAM3, 3, 8, W.sam3_hparams(), [("huge4", orc.F32, (big, big), np.zeros(8, np.uint8))])
    _expect_error(mi, p, -3)                                        # 4 * count past int64
    W.write(p, W.MAGIC_SAM3, 3, 8, W.sam3_hparams(), [("long", orc.F32, (2**30, 2**29), np.zeros(8, np.uint8))])
    _expect_error(mi, p, -1)                                        # 2^61 bytes in a tiny file


def test_corrupted_files_fail_cleanly(mi, orc, tmp_path):
    """Seeded byte mutations of a valid file (header, hyperparameters and tensor
    records, where lengths, dims and types live): opening either succeeds with
    a consistent index or raises the library's error; it never crashes, hangs
    or allocates beyond the file.  Runs in a child process so that a crash
    would fail the test instead of ending the session."""
    import subprocess, sys, textwrap
    p = tmp_path / "m.ggml"
    W.write(p, W.MAGIC_SAM3, 3, 8, W.sam3_hparams(), _tensors(orc))
    code = textwrap.dedent(f"""
        import importlib.util, os, numpy as np, resource
        resource.setrlimit(resource.RLIMIT_AS, (8 << 30, 8 << 30))
        spec = importlib.util.spec_from_file_location("m", {str(mi.__file__)!r})
        mi = importlib.util.module_from_spec(spec); spec.loader.exec_module(mi)
        src = open({str(p)!r}, "rb").read()
        rng = np.random.default_rng(11)
        out = {str(tmp_path / "x.ggml")!r}
        ok = err = 0
        head = min(len(src), 1024)  # header, hparams and the first tensor records
        for i in range(400):
            b = bytearray(src)
            for _ in range(int(rng.integers(1, 4))):
                j = int(rng.integers(0, head))
                b[j] = int(rng.integers(0, 256))
            open(out, "wb").write(bytes(b))
            try:
                f = mi.ModelFile(out)
                for t in range(f.header()[3]):
                    info = f.tensor(t)
                    assert info["offset"] + info["nbytes"] <= len(b), (info, len(b))
                f.close()
                ok += 1
            except mi.Mi355Error:
                err += 1
        print(ok, err)
    """)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    ok, err = map(int, r.stdout.split())
    assert ok + err == 400 and err > 0
