"""Benchmark of the quantized mul_mat hot path on one MI355X.

Workload ("step"): the SAM3 ViT block linear set at 72x72 = 5184 tokens --
qkv [3072x1024], attn-out [1024x1024], fc1 [4736x1024], fc2 [1024x4736] --
once with Q8_0 weights and once with Q4_0 weights (8 ggml mul_mat calls,
each quantizing its f32 activations to one-byte Q8_0 quants and running the
int8 MFMA GEMM).  Weights are quantized from f32 N(0,0.02) and prepared once
at setup (mi355_weight_prepare, as a model load would); activations f32
N(0,1) (seed 0), one buffer per call so that no call re-reads another's
activations from the last-level cache; all inputs are resident in HBM before
timing.  The same calls with the weights in the ggml layout (repacked on
every call) are timed after the step and reported as raw_layout_tops.

value = int8 ops of the step (2*M*N*K per GEMM) / step time, in TOPS.

Also reported: per-type TOPS and %% of the int8 dense MFMA peak, the
dominant kernel's roofline (the fc1 Q8_0 MMQ kernel, timed with HIP events
on its stream through the library's kernel-timing hook), and a CPU baseline
(the oracle's ggml-cpu restatement of the same mul_mat, AVX2 or AVX512-VNNI, on the host;
beside it the SAM3 ViT encoder per frame from one windowed and one global
block of the oracle's block composition, extrapolated x28 / x4).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

INT8_PEAK_TOPS = 5033.0      # MI355X dense int8 MFMA (256 CU x 2.4 GHz x 8192 op/clk/CU)
FP16_PEAK_TFLOPS = 2516.0    # MI355X dense fp16 MFMA
HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
M_TOK = 5184
LINEARS = [("qkv", 3072, 1024), ("proj", 1024, 1024), ("fc1", 4736, 1024), ("fc2", 1024, 4736)]
TYPES = ["q8_0", "q4_0"]
CONFIG2_TYPES = ["q4_1", "f16"]  # config 2's other weight types, reported beside the step
ALL_TYPES = ["q8_0", "q4_0", "q4_1", "f16"]


# the oracle's dot-product paths (orc_isa_path): AVX2, or AVX2 with AVX512-VNNI for the quantized dots
ISA_NAMES = {0: "scalar", 1: "avx2", 2: "avx512vnni"}

PREWARM_S = 0.5  # seconds of back-to-back work before each timed section (--prewarm)


def prewarm(fn, torch, seconds=None):
    """Runs fn back to back for `seconds` of wall time: a GPU that has been idle
    (host-side input generation, weight preparation) runs its first ~100 ms of
    work at reduced clocks, and the timed sections measure the sustained state
    an encoder serving a stream of frames runs in.  The inputs stay the timed
    section's own, so nothing is cached that the timed calls would not see."""
    seconds = PREWARM_S if seconds is None else seconds
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        fn()
        torch.cuda.synchronize()


def cpu_model() -> str:
    """The host CPU's model string (/proc/cpuinfo), or "unknown"."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def load_pkg():
    import importlib.util
    spec = importlib.util.spec_from_file_location("sam3_cpp_amd", os.path.join(ROOT, "sam3.cpp_amd", "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["sam3_cpp_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def _pmc_run(counter, op, kernel_sub):
    """Average per-dispatch value (KiB) of one TCC byte counter for the
    dispatches of kernels whose name contains kernel_sub, from a child
    `rocprofv3 --pmc` run of this script in --op mode."""
    import csv
    import shutil
    import subprocess
    import tempfile
    prof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    with tempfile.TemporaryDirectory(dir="/tmp") as td:
        cmd = [prof, "--pmc", counter, "--output-format", "csv", "-d", td, "-o", "run", "--",
               sys.executable, os.path.abspath(__file__), "--op", op, "--reps", "5", "--op-warmup", "3"]
        env = dict(os.environ, TMPDIR="/tmp")
        subprocess.run(cmd, cwd="/tmp", env=env, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL,
                       timeout=150, check=True)
        vals = []
        for root, _, files in os.walk(td):
            for f in files:
                if f.endswith("counter_collection.csv"):
                    for r in csv.DictReader(open(os.path.join(root, f))):
                        if kernel_sub in r["Kernel_Name"] and r["Counter_Name"] == counter:
                            vals.append(float(r["Counter_Value"]))
        if not vals:
            raise RuntimeError(f"no {counter} samples for {kernel_sub}")
        return sum(vals) / len(vals)


def measure_traffic(op, kernel_sub):
    """HBM bytes per launch of the op's kernel: FETCH_SIZE and WRITE_SIZE
    (KiB per dispatch), each scaled by what the same counter reads for a plain
    256 MiB device copy (read 256 MiB, write 256 MiB)."""
    copy_bytes = 256 << 20
    f_copy = _pmc_run("FETCH_SIZE", "copy", "copyBuffer")
    w_copy = _pmc_run("WRITE_SIZE", "copy", "copyBuffer")
    f = _pmc_run("FETCH_SIZE", op, kernel_sub)
    w = _pmc_run("WRITE_SIZE", op, kernel_sub)
    fs, ws = copy_bytes / (f_copy * 1024), copy_bytes / (w_copy * 1024)
    return {"bytes": round(f * 1024 * fs + w * 1024 * ws), "fetch_kib": round(f, 1), "write_kib": round(w, 1),
            "fetch_scale": round(fs, 4), "write_scale": round(ws, 4)}


def bench_attention(mi, ctx, torch, dev, only=None, reps=20):
    """FLASH_ATTN_EXT at the SAM3 shapes: f16 Q/K/V N(0,1), head 64, 16 heads;
    windowed = 9 windows of 576 tokens (batch 144), global = 5184 tokens."""
    res = {}
    g = torch.Generator(device=dev).manual_seed(0)
    for name, n, B in (("windowed", 576, 9), ("global", 5184, 1)):
        if only and name != only:
            continue
        D, nh = 64, 16
        q, k, v = (torch.randn((B, nh, n, D), generator=g, device=dev).half() for _ in range(3))
        dst = torch.empty((B, n, nh, D), dtype=torch.float32, device=dev)
        tq, tk, tv = (mi.from_torch(x, mi.F16, [D, n, nh, B]) for x in (q, k, v))
        td = mi.from_torch(dst, mi.F32, [D, nh, n, B])
        prewarm(lambda: ctx.flash_attn_ext(tq, tk, tv, td, 0.125), torch)
        for _ in range(5):
            ctx.flash_attn_ext(tq, tk, tv, td, 0.125)
        torch.cuda.synchronize()
        ctx.profile(True)
        for _ in range(reps):
            ctx.flash_attn_ext(tq, tk, tv, td, 0.125)
        pr = ctx.profile_collect()
        ctx.profile(False)
        us = 1e3 * pr["flash_attn_ext"][1] / pr["flash_attn_ext"][0]
        flop = 4.0 * B * nh * n * n * D
        res[name] = {"us": round(us, 2), "tflops": round(flop / us / 1e6, 1),
                     "pct_fp16_peak": round(100 * flop / us / 1e6 / FP16_PEAK_TFLOPS, 2)}
    return res


def prepare_weight(mi, ctx, torch, dev, wt, keep):
    """wt prepared once (mi355_weight_prepare) into a new device buffer, as a model load would."""
    n = mi.weight_prepared_nbytes(wt)
    buf = torch.empty(n + 256, dtype=torch.uint8, device=dev)
    keep.append(buf)
    return ctx.weight_prepare(wt, buf.data_ptr() + (-buf.data_ptr()) % 256, n)


def vit_block_host(orc, i, seed=0):
    """Block i's f32 vectors (LayerNorm weights near 1, biases N(0, 0.02)) and
    f32 N(0, 0.02) linear weights [out][in], as host arrays."""
    E, MLP = 1024, 4736
    vec = {}
    for j, (name, n, sc, m) in enumerate([("norm1_w", E, 0.1, 1.0), ("norm1_b", E, 0.02, 0.0),
                                          ("qkv_b", 3 * E, 0.02, 0.0), ("proj_b", E, 0.02, 0.0),
                                          ("norm2_w", E, 0.1, 1.0), ("norm2_b", E, 0.02, 0.0),
                                          ("fc1_b", MLP, 0.02, 0.0), ("fc2_b", E, 0.02, 0.0)]):
        vec[name] = orc.normal(n, seed + i, 200 + j) * np.float32(sc) + np.float32(m)
    ws = {}
    for j, (name, n, k) in enumerate([("qkv", 3 * E, E), ("proj", E, E), ("fc1", MLP, E), ("fc2", E, MLP)]):
        ws[name] = (orc.normal(n * k, seed + i, 100 + j, std=0.02).reshape(n, k), n, k)
    return vec, ws


def cpu_encoder_baseline(orc, tname, reps, warmup):
    """SAM3 ViT encoder time per 1008^2 frame on the host cores, from the
    oracle's composition of sam3_vit_block_forward (ggml-cpu's algorithms:
    quantized mul_mat with Q8_0 activations, F32 flash attention, LayerNorm,
    RoPE, GELU-erf): one windowed block (block 0) and one global block
    (block 7) on N(0, 1) tokens, extrapolated as 28 windowed + 4 global
    blocks, the extrapolation of tests/test_metal_overhead.cpp:249-252.
    Each block time is the median of reps runs after warmup runs."""
    from oracle import blocks as ob
    E, NH, MLP, WS, G = 1024, 16, 4736, 24, 72
    t = orc.NAME_TYPE[tname]
    x = orc.normal(G * G * E, 0, 310).reshape(G * G, E)
    res = {}
    for name, i, glob in (("windowed", 0, False), ("global", 7, True)):
        vec, ws = vit_block_host(orc, i)
        host = {k: (orc.quantize_weights(t, w), n, kk) for k, (w, n, kk) in ws.items()}
        freqs = ob.axial_cis(orc, E // NH, G, WS / G) if glob else ob.axial_cis(orc, E // NH, WS, 1.0)
        times = []
        for r in range(warmup + reps):
            t0 = time.perf_counter()
            out = ob.vit_block_ref(orc, t, x, host, vec, E, NH, MLP, G, 0 if glob else WS, freqs, False)
            if r >= warmup:
                times.append(time.perf_counter() - t0)
        if not np.isfinite(out).all():
            raise RuntimeError("cpu encoder baseline: non-finite block output")
        res[name] = float(np.median(times))
    frame = 28 * res["windowed"] + 4 * res["global"]
    nth = orc.nthreads()
    return {"ms_per_frame": round(frame * 1e3, 1), "windowed_block_ms": round(res["windowed"] * 1e3, 1),
            "global_block_ms": round(res["global"] * 1e3, 1), "cores": nth, "kind": "port",
            "sample": f"{tname} SAM3 ViT: one windowed and one global block (median of {reps} after {warmup} "
                      f"warmups each), x28 + x4; {nth} threads of nproc={os.cpu_count()}, "
                      f"isa={ISA_NAMES.get(orc.lib().orc_isa_path(), 'scalar')}, cpu={cpu_model()}"}


def build_encoder(mi, orc, torch, dev, types, seed=0, ctx=None):
    """Random-init SAM3 ViT (1008^2 image, patch 14, E 1024, 32 blocks, 16 heads,
    MLP 4736, windows of 24 except global blocks 7/15/23/31): per type, the
    32 blocks' linear weights quantized from the same f32 N(0,0.02) draws and,
    with a context, prepared for the int8 kernel."""
    E, NH, MLP, WS, G, P, PG = 1024, 16, 4736, 24, 72, 14, 24
    HD = E // NH
    hp = mi.VitHparams(E, NH, MLP, WS, G, P, PG, 1e-5)
    keep = []

    def up(a):
        t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
        keep.append(t)
        return t

    def cis(end, scale):
        out = np.empty(end * end * HD, dtype=np.float32)
        orc.lib().orc_compute_axial_cis(out.ctypes.data, HD, end, end, C.c_float(10000.0), C.c_float(scale))
        return up(out)

    f_win, f_glob = cis(WS, 1.0), cis(G, WS / G)
    blocks = {tn: [] for tn in types}
    for i in range(32):
        glob = i in (7, 15, 23, 31)
        vec_h, ws = vit_block_host(orc, i, seed)
        vec = {name: up(a) for name, a in vec_h.items()}
        for tn in types:
            t = orc.NAME_TYPE[tn]
            blk = mi.VitBlock()
            for name, (w, n, k) in ws.items():
                wt = mi.from_torch(up(orc.quantize_weights(t, w)), t, [k, n])
                if ctx is not None and mi.weight_prepared_nbytes(wt):
                    wt = prepare_weight(mi, ctx, torch, dev, wt, keep)
                setattr(blk, name + "_w", wt)
            for name, tsr in vec.items():
                setattr(blk, name, tsr.data_ptr())
            blk.freqs_cis = (f_glob if glob else f_win).data_ptr()
            blk.is_global = 1 if glob else 0
            blocks[tn].append(blk)
    image = up(orc.uniform(3 * 1008 * 1008, seed, 300).reshape(3, 1008, 1008))
    patch_w = up(orc.normal(E * 3 * P * P, seed, 301, std=0.02))
    pos = up(orc.normal(PG * PG * E, seed, 302, std=0.02))
    ln_w = up(orc.normal(E, seed, 303) * np.float32(0.1) + np.float32(1.0))
    ln_b = up(orc.normal(E, seed, 304) * np.float32(0.02))
    pre = (image.data_ptr(), mi.from_torch(patch_w, mi.F32, [P, P, 3, E]), pos.data_ptr(), ln_w.data_ptr(),
           ln_b.data_ptr())
    return hp, pre, blocks, keep


def build_hiera(mi, orc, torch, dev, tname, seed=0, ctx=None):
    """Random-init SAM2.1 Hiera-tiny (img 1024, embed 96, heads 1, stages
    1/2/7/2, windows 8/4/14/7, global blocks 5/7/9, q_pool 3): linear weights
    f32 N(0,0.02) quantized to tname; the patch weight is F16 under F16 weights
    and F32 otherwise (its rows of 7 are not a multiple of 32)."""
    t = orc.NAME_TYPE[tname]
    hp = mi.hiera_tiny(1024)
    keep = []

    def up(a):
        x = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
        keep.append(x)
        return x

    blocks = []
    for i in range(mi.lib().mi355_hiera_n_blocks(hp)):
        info = mi.hiera_block_info(hp, i)
        cin, cout = info.dim_in, info.dim_out
        blk = mi.HieraBlock()
        shapes = [("qkv", 3 * cout, cin), ("proj", cout, cout), ("fc1", 4 * cout, cout), ("fc2", cout, 4 * cout)]
        if cin != cout:
            shapes.append(("dim_proj", cout, cin))
        for j, (name, n, k) in enumerate(shapes):
            w = orc.normal(n * k, seed + i, 400 + j, std=0.02).reshape(n, k)
            wt = mi.from_torch(up(orc.quantize_weights(t, w)), t, [k, n])
            if ctx is not None and mi.weight_prepared_nbytes(wt):
                wt = prepare_weight(mi, ctx, torch, dev, wt, keep)
            setattr(blk, name + "_w", wt)
        for j, (name, n, sc, m) in enumerate([("norm1_w", cin, 0.1, 1.0), ("norm1_b", cin, 0.02, 0.0),
                                              ("qkv_b", 3 * cout, 0.02, 0.0), ("proj_b", cout, 0.02, 0.0),
                                              ("norm2_w", cout, 0.1, 1.0), ("norm2_b", cout, 0.02, 0.0),
                                              ("fc1_b", 4 * cout, 0.02, 0.0), ("fc2_b", cout, 0.02, 0.0),
                                              ("dim_proj_b", cout, 0.02, 0.0)]):
            setattr(blk, name, up(orc.normal(n, seed + i, 450 + j) * np.float32(sc) + np.float32(m)).data_ptr())
        blocks.append(blk)
    E, S0 = hp.embed_dim, hp.img_size // 4
    image = up(orc.uniform(3 * hp.img_size ** 2, seed, 500).reshape(3, hp.img_size, hp.img_size))
    pw32 = orc.normal(E * 147, seed, 501, std=0.02)
    if t == orc.F16:
        patch_w = mi.from_torch(up(orc.quantize_weights(orc.F16, pw32.reshape(E, 147))), mi.F16, [7, 7, 3, E])
    else:
        patch_w = mi.from_torch(up(pw32), mi.F32, [7, 7, 3, E])
    patch_b = up(orc.normal(E, seed, 502) * np.float32(0.02))
    pos = up(orc.normal(S0 * S0 * E, seed, 503, std=0.02))
    dims, S, stage_dims = [], S0, []
    for i in range(len(blocks)):
        info = mi.hiera_block_info(hp, i)
        if info.q_stride:
            S //= 2
        dims.append((S, info.dim_out, info.stage))
    for st in range(4):
        last = [d for d in dims if d[2] == st][-1]
        stage_dims.append((last[0], last[1]))
    outs = [torch.empty((s * s, c), dtype=torch.float32, device=dev) for s, c in stage_dims]
    keep += outs
    return hp, (image.data_ptr(), patch_w, patch_b.data_ptr(), pos.data_ptr()), blocks, outs, keep


def bench_hiera(mi, ctx, torch, hp, pre, blocks, outs, frames):
    """ms per frame of the Hiera-tiny backbone (patch embedding + 12 blocks),
    image resident in HBM; plus one profiled frame split by kernel."""
    img, pw, pb, pos = pre
    ptrs = [o.data_ptr() for o in outs]
    run = lambda: ctx.hiera_encode(hp, C.c_void_p(img), pw, C.c_void_p(pb), C.c_void_p(pos), blocks, ptrs)
    prewarm(run, torch)
    run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(frames):
        run()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / frames
    finite = all(bool(torch.isfinite(o).all().item()) for o in outs)
    ctx.profile(True)
    run()
    pr = ctx.profile_collect()
    ctx.profile(False)
    split = {k: round(v[1], 3) for k, v in sorted(pr.items(), key=lambda kv: -kv[1][1])}
    return {"ms_per_frame": round(ms, 3), "frames": frames, "output_finite": finite, "kernel_ms_per_frame": split}


def build_neck(mi, orc, torch, dev, tname, seed=0):
    """SAM3 SimpleFPN neck at 1008^2: ViT output [72*72][1024] N(0,1), E = 1024,
    C1 = 512, D = 256; kernels N(0, 0.02) in F32 (their type under quantized
    ftypes) or F16, biases N(0, 0.02)."""
    E, C1, D, G = 1024, 512, 256, 72
    t = orc.NAME_TYPE[tname]
    keep = []

    def up(a):
        x = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
        keep.append(x)
        return x

    def kern(j, n_el, ne):
        w = orc.normal(n_el, seed, 600 + j, std=0.02)
        if t == orc.F16:
            w = w.astype(np.float16).view(np.uint16)
        k = mi.from_torch(up(w), t, ne)
        keep.append(k)
        return k

    def bias(j, n):
        return up(orc.normal(n, seed, 650 + j, std=0.02)).data_ptr()

    sc = [dict(deconv1_w=kern(0, 4 * C1 * E, [2, 2, C1, E]), deconv1_b=bias(0, C1),
               deconv2_w=kern(1, 4 * D * C1, [2, 2, D, C1]), deconv2_b=bias(1, D),
               conv1x1_w=kern(2, D * D, [1, 1, D, D]), conv1x1_b=bias(2, D),
               conv3x3_w=kern(3, 9 * D * D, [3, 3, D, D]), conv3x3_b=bias(3, D)),
          dict(deconv1_w=kern(4, 4 * C1 * E, [2, 2, C1, E]), deconv1_b=bias(4, C1),
               conv1x1_w=kern(5, D * C1, [1, 1, C1, D]), conv1x1_b=bias(5, D),
               conv3x3_w=kern(6, 9 * D * D, [3, 3, D, D]), conv3x3_b=bias(6, D))]
    for i in range(2):
        sc.append(dict(conv1x1_w=kern(7 + 2 * i, D * E, [1, 1, E, D]), conv1x1_b=bias(7 + 2 * i, D),
                       conv3x3_w=kern(8 + 2 * i, 9 * D * D, [3, 3, D, D]), conv3x3_b=bias(8 + 2 * i, D)))
    x = up(orc.normal(G * G * E, seed, 660))
    outs = [torch.empty((n, D), dtype=torch.float32, device=dev) for n in (16 * G * G, 4 * G * G, G * G, G * G // 4)]
    keep += outs
    return (E, G), sc, x, outs, keep


def neck_flops(E=1024, C1=512, D=256, G=72):
    """Multiply-add work of one neck (2 per MAC): conv-transposes, 1x1, 3x3."""
    P = G * G
    dec = 2 * (P * E * 4 * C1 + 4 * P * C1 * 4 * D + P * E * 4 * C1)
    c1 = 2 * (16 * P * D * D + 4 * P * C1 * D + P * E * D + P // 4 * E * D)
    c3 = 2 * 9 * D * D * (16 * P + 4 * P + P + P // 4)
    return dec + c1 + c3


def bench_neck(mi, ctx, torch, dims, sc, x, outs, frames):
    """ms per SimpleFPN neck (four maps from the ViT output), inputs resident in
    HBM; plus one profiled run split by kernel."""
    E, G = dims
    ptrs = [o.data_ptr() for o in outs]
    run = lambda: ctx.sam3_neck(x.data_ptr(), E, G, sc, ptrs)
    prewarm(run, torch)
    run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(frames):
        run()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / frames
    finite = all(bool(torch.isfinite(o).all().item()) for o in outs)
    ctx.profile(True)
    run()
    pr = ctx.profile_collect()
    ctx.profile(False)
    split = {k: round(v[1], 3) for k, v in sorted(pr.items(), key=lambda kv: -kv[1][1])}
    fl = neck_flops()
    return {"ms_per_neck": round(ms, 3), "frames": frames, "tflops": round(fl / (ms * 1e-3) / 1e12, 1),
            "gflop": round(fl / 1e9, 1), "output_finite": finite, "kernel_ms": split}


def bench_encoder(mi, ctx, torch, dev, hp, pre, blocks, frames):
    """ms per frame of the whole encoder (prefix + 32 blocks), image resident in
    HBM; plus one profiled frame split by kernel."""
    x = torch.empty((hp.grid * hp.grid, hp.embed_dim), dtype=torch.float32, device=dev)
    img, pw, pos, lw, lb = pre
    run = lambda: ctx.vit_encode(hp, C.c_void_p(img), pw, C.c_void_p(pos), C.c_void_p(lw), C.c_void_p(lb), blocks,
                                 C.c_void_p(x.data_ptr()))
    prewarm(run, torch)
    run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(frames):
        run()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / frames
    finite = bool(torch.isfinite(x).all().item())
    ctx.profile(True)
    run()
    pr = ctx.profile_collect()
    ctx.profile(False)
    split = {k: round(v[1], 3) for k, v in sorted(pr.items(), key=lambda kv: -kv[1][1])}
    return {"ms_per_frame": round(ms, 3), "frames": frames, "output_finite": finite, "kernel_ms_per_frame": split}


def main():
    global PREWARM_S
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-encoder-reps", type=int, default=3,
                    help="CPU encoder baseline: timed runs per block (median), 0 to skip")
    ap.add_argument("--cpu-encoder-warmup", type=int, default=1, help="CPU encoder baseline: untimed runs per block")
    ap.add_argument("--no-encoder", action="store_true", help="skip the full ViT encoder ms/frame")
    ap.add_argument("--frames", type=int, default=3, help="timed encoder frames per weight type")
    ap.add_argument("--op", default=None,
                    help="profile mode, one workload --reps times with its kernel times: TYPE/LINEAR (e.g. q8_0/fc1), "
                         "attn/windowed, attn/global, vit/TYPE (SAM3 ViT frames), hiera/TYPE (Hiera-tiny frames), "
                         "neck/f32|f16 (SAM3 SimpleFPN neck), mm/TYPE/MxNxK (one MUL_MAT of that shape, "
                         "e.g. mm/q4_0/65536x288x96 for the SAM2 Hiera-tiny stage-1 qkv), "
                         "copy (256 MiB device copy)")
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--op-warmup", type=int, default=20)
    ap.add_argument("--prewarm", type=float, default=PREWARM_S,
                    help="seconds of back-to-back untimed work before each timed section (GPU clocks at their "
                         "sustained level)")
    ap.add_argument("--mmq-kernel", choices=["auto", "f16", "int8"], default="auto",
                    help="kernel of MUL_MATs with ggml-layout Q8_0/Q4_0/Q4_1 weights (mi355_context_set_mmq_kernel)")
    ap.add_argument("--raw-weights", action="store_true",
                    help="encoders: quantized weights in the ggml layout (fp16 kernels) instead of prepared")
    ap.add_argument("--no-fuse", action="store_true",
                    help="encoder modes: run the unfused pass sequence (f32 activations between the ggml node groups)")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the rocprofv3 FETCH_SIZE/WRITE_SIZE child runs (roofline.traffic = null)")
    args = ap.parse_args()
    PREWARM_S = args.prewarm
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "the hot path shards over tokens or frames, one process per GPU, with no collective "
              "inside a MUL_MAT", file=sys.stderr)
        sys.exit(2)

    traffic = None
    if not args.op and not args.no_traffic:
        # child profiler runs first, before this process initialises the GPU
        log("bench: HBM traffic of mmq_q8_0 fc1 (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)")
        try:
            traffic = measure_traffic("q8_0/fc1", "mmq8_kernel<8")
        except Exception as e:  # profiler missing or failed: traffic stays unmeasured
            log(f"bench: traffic measurement failed: {e!r}")

    import torch
    from oracle import oracle as orc

    mi = load_pkg()
    ctx = mi.Context(0)
    ctx.set_mmq_kernel({"auto": mi.MMQ_AUTO, "f16": mi.MMQ_F16, "int8": mi.MMQ_INT8}[args.mmq_kernel])
    dev = torch.device("cuda:0")

    if args.op == "copy":
        # calibration for the HBM byte counters: a plain device copy of 256 MiB
        # (reads 256 MiB, writes 256 MiB per launch)
        n = 64 << 20
        a = torch.empty(n, dtype=torch.float32, device=dev).uniform_()
        b = torch.empty_like(a)
        for _ in range(args.reps):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"op": "copy", "bytes_read": 4 * n, "bytes_written": 4 * n, "reps": args.reps}), flush=True)
        ctx.close()
        return

    if args.op and args.op.startswith("attn/"):
        which = args.op.split("/")[1]
        res = bench_attention(mi, ctx, torch, dev, only=which, reps=args.reps)
        print(json.dumps({"op": args.op, "reps": args.reps, **res[which]}), flush=True)
        ctx.close()
        return
    if args.no_fuse:
        ctx.set_fusion(False)
    if args.op and args.op.startswith("hiera/"):
        tn = args.op.split("/")[1]
        hp, pre, blocks, outs, keep = build_hiera(mi, orc, torch, dev, tn, ctx=None if args.raw_weights else ctx)
        res = bench_hiera(mi, ctx, torch, hp, pre, blocks, outs, args.reps)
        print(json.dumps({"op": args.op, **res}), flush=True)
        ctx.close()
        return
    if args.op and args.op.startswith("mm/"):
        _, tn, shape = args.op.split("/")
        M, N, K = (int(v) for v in shape.split("x"))
        t = orc.NAME_TYPE[tn]
        w = orc.normal(N * K, seed=0, stream=70, std=0.02).reshape(N, K)
        wd = torch.from_numpy(orc.quantize_weights(t, w)).to(dev)
        xm = torch.from_numpy(orc.normal(M * K, seed=0, stream=71).reshape(M, K)).to(dev)
        dst = torch.empty((M, N), dtype=torch.float32, device=dev)
        s0, s1 = mi.from_torch(wd, t, [K, N]), mi.from_torch(xm, mi.F32, [K, M])
        keep_w = []
        if not args.raw_weights and mi.weight_prepared_nbytes(s0):
            s0 = prepare_weight(mi, ctx, torch, dev, s0, keep_w)  # as the bench step's weights
        d = mi.from_torch(dst, mi.F32, [N, M])
        prewarm(lambda: ctx.mul_mat(s0, s1, d), torch)
        for _ in range(args.op_warmup):
            ctx.mul_mat(s0, s1, d)
        torch.cuda.synchronize()
        ctx.profile(True)
        for _ in range(args.reps):
            ctx.mul_mat(s0, s1, d)
        prof = ctx.profile_collect()
        ctx.profile(False)
        print(json.dumps({"op": args.op, "reps": args.reps,
                          "kernel_us": {k: round(1e3 * v[1] / v[0], 2) for k, v in prof.items()}}), flush=True)
        ctx.close()
        return
    if args.op and args.op.startswith("neck/"):
        tn = args.op.split("/")[1]
        dims, sc, x, outs, keep = build_neck(mi, orc, torch, dev, tn)
        res = bench_neck(mi, ctx, torch, dims, sc, x, outs, args.reps)
        print(json.dumps({"op": args.op, **res}), flush=True)
        ctx.close()
        return
    if args.op and args.op.startswith("vit/"):
        tn = args.op.split("/")[1]
        hp, pre, blocks, keep = build_encoder(mi, orc, torch, dev, [tn], ctx=None if args.raw_weights else ctx)
        res = bench_encoder(mi, ctx, torch, dev, hp, pre, blocks[tn], args.reps)
        print(json.dumps({"op": args.op, **res}), flush=True)
        ctx.close()
        return

    # ---- inputs (host-generated with the counter RNG, then resident in HBM)
    log("bench: generating inputs")
    x1024 = orc.normal(M_TOK * 1024, seed=0, stream=2).reshape(M_TOK, 1024)
    x4736 = orc.normal(M_TOK * 4736, seed=0, stream=3).reshape(M_TOK, 4736)
    xhost = {1024: x1024, 4736: x4736}
    calls = []  # (tname, lname, N, K, s0 prepared, s1, d, s0 in the ggml layout)
    host_w = {}
    keep = []
    types = TYPES + CONFIG2_TYPES  # the step's types, then config 2's Q4_1 / F16 (timed per call only)
    if args.op:
        types = [args.op.split("/")[0]]
    for ti, tname in enumerate(types):
        t = orc.NAME_TYPE[tname]
        for li, (lname, N, K) in enumerate(LINEARS):
            w = orc.normal(N * K, seed=0, stream=10 + li, std=0.02).reshape(N, K)
            wq = orc.quantize_weights(t, w)
            host_w[(tname, lname)] = wq
            wd = torch.from_numpy(wq).to(dev)
            wt = mi.from_torch(wd, t, [K, N])
            nbw = mi.weight_prepared_nbytes(wt)  # 0 for F16 weights: those run as given
            wbuf = torch.empty(nbw + 256, dtype=torch.uint8, device=dev)
            s0 = ctx.weight_prepare(wt, wbuf.data_ptr() + (-wbuf.data_ptr()) % 256, nbw) if nbw else wt
            wbuf = (wbuf, wd)
            xd = torch.from_numpy(xhost[K]).to(dev)  # this call's own activations
            dst = torch.empty((M_TOK, N), dtype=torch.float32, device=dev)
            s1 = mi.from_torch(xd, mi.F32, [K, M_TOK])
            d = mi.from_torch(dst, mi.F32, [N, M_TOK])
            keep.append((wbuf, xd))
            calls.append((tname, lname, N, K, s0, s1, d, wt))
    ctx.synchronize()
    if args.op:
        c = [c for c in calls if f"{c[0]}/{c[1]}" == args.op][0]
        prewarm(lambda: ctx.mul_mat(c[4], c[5], c[6]), torch)
        for _ in range(args.op_warmup):
            ctx.mul_mat(c[4], c[5], c[6])
        torch.cuda.synchronize()
        ctx.profile(True)
        for _ in range(args.reps):
            ctx.mul_mat(c[4], c[5], c[6])
        prof = ctx.profile_collect()
        print(json.dumps({"op": args.op, "reps": args.reps,
                          "kernel_us": {k: round(1e3 * v[1] / v[0], 2) for k, v in prof.items()}}), flush=True)
        ctx.close()
        return
    ops_by_type = {tn: sum(2.0 * M_TOK * N * K for (_, N, K) in LINEARS) for tn in TYPES + CONFIG2_TYPES}
    step_ops = sum(ops_by_type[tn] for tn in TYPES)
    extra_calls = [c for c in calls if c[0] in CONFIG2_TYPES]
    calls = [c for c in calls if c[0] in TYPES]

    def step():
        for c in calls:
            ctx.mul_mat(c[4], c[5], c[6])

    # ---- timed region
    log("bench: warmup")
    prewarm(step, torch)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    log(f"bench: timing {args.steps} steps")
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms_step = e0.elapsed_time(e1) / args.steps

    # per-type and per-kernel times with the library's event hook
    ctx.profile(True)
    per_call_ms = {}
    for c in calls:
        for _ in range(5):
            ctx.mul_mat(c[4], c[5], c[6])
        prof = ctx.profile_collect()
        per_call_ms[(c[0], c[1])] = {k: v[1] / v[0] for k, v in prof.items()}
    ctx.profile(False)
    log("bench: per-call kernel times " + json.dumps({f"{a}/{b}": v for (a, b), v in per_call_ms.items()}))
    # the same calls with the weights in the ggml layout (the int8 route repacks them on each call)
    ctx.profile(True)
    raw_call_ms = {}
    for c in calls:
        for _ in range(5):
            ctx.mul_mat(c[7], c[5], c[6])
        prof = ctx.profile_collect()
        raw_call_ms[(c[0], c[1])] = {k: v[1] / v[0] for k, v in prof.items()}
    ctx.profile(False)
    log("bench: per-call kernel times, ggml-layout weights " +
        json.dumps({f"{a}/{b}": v for (a, b), v in raw_call_ms.items()}))

    # config 2's other weight types over the same linear set: Q4_1 (prepared, int8 kernel) and F16
    # (fp16 MFMA kernel), per-call kernel times after a pre-warm
    cfg2 = {}
    for tname in CONFIG2_TYPES:
        tc = [c for c in extra_calls if c[0] == tname]
        prewarm(lambda: [ctx.mul_mat(c[4], c[5], c[6]) for c in tc], torch)
        ctx.profile(True)
        per = {}
        for c in tc:
            for _ in range(5):
                ctx.mul_mat(c[4], c[5], c[6])
            prof = ctx.profile_collect()
            per[c[1]] = {k: round(1e3 * v[1] / v[0], 2) for k, v in prof.items()}
        ctx.profile(False)
        tot_ms = sum(sum(v.values()) for v in per.values()) * 1e-3
        cfg2[tname] = {"tops": round(ops_by_type[tname] / (tot_ms * 1e-3) / 1e12, 2), "kernel_us": per,
                       "weights": "prepared" if tname != "f16" else "as given (F16)"}
    log("bench: config 2 Q4_1 / F16 " + json.dumps(cfg2))

    type_tops, raw_tops = {}, {}
    for tname in TYPES:
        tot = sum(sum(per_call_ms[(tname, ln)].values()) for (ln, _, _) in LINEARS)
        type_tops[tname] = ops_by_type[tname] / (tot * 1e-3) / 1e12
        tot = sum(sum(raw_call_ms[(tname, ln)].values()) for (ln, _, _) in LINEARS)
        raw_tops[tname] = ops_by_type[tname] / (tot * 1e-3) / 1e12

    # ---- roofline of the dominant kernel: MMQ Q8_0 at the fc1 shape
    N, K = 4736, 1024
    mmq_ms = per_call_ms[("q8_0", "fc1")]["mmq8_q8_0"]
    w_bytes = N * (K // 32) * 34
    a_bytes = M_TOK * K + M_TOK * (K // 32) * 4      # int8 activation quants + scale dwords
    d_bytes = M_TOK * N * 4
    alg_bytes = w_bytes + a_bytes + d_bytes
    achieved = alg_bytes / (mmq_ms * 1e-3) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": traffic["bytes"] if traffic else None,
                "kernel": "mmq8_q8_0 fc1 [5184x1024]x[4736x1024]", "kernel_us": round(mmq_ms * 1e3, 2),
                "alg_bytes": alg_bytes,
                "traffic_counters": traffic,
                "int8_tops": round(2.0 * M_TOK * N * K / (mmq_ms * 1e-3) / 1e12, 1)}

    # ---- attention (FLASH_ATTN_EXT at the windowed / global SAM3 shapes)
    log("bench: attention")
    attn = bench_attention(mi, ctx, torch, dev)

    # ---- full SAM3 ViT encoder ms/frame, Q8_0 and Q4_0 weights
    encoder = None
    hiera = None
    neck_res = None
    if not args.no_encoder:
        log("bench: encoder weights")
        del calls, extra_calls, keep
        torch.cuda.empty_cache()
        hp, pre, blocks, keep = build_encoder(mi, orc, torch, dev, TYPES, ctx=None if args.raw_weights else ctx)
        encoder = {}
        for tn in TYPES:
            log(f"bench: encoder {tn}")
            encoder[tn] = bench_encoder(mi, ctx, torch, dev, hp, pre, blocks[tn], args.frames)
        del keep
        hiera = {}
        for tn in ("f16", "q4_0"):
            log(f"bench: hiera-tiny {tn}")
            hp_h, pre_h, blocks_h, outs_h, keep_h = build_hiera(mi, orc, torch, dev, tn, ctx=None if args.raw_weights else ctx)
            hiera[tn] = bench_hiera(mi, ctx, torch, hp_h, pre_h, blocks_h, outs_h, 5)
            del keep_h
        neck_res = {}
        for tn in ("f32", "f16"):
            log(f"bench: neck {tn}")
            dims, sc, xn, outs_n, keep_n = build_neck(mi, orc, torch, dev, tn)
            neck_res[tn] = bench_neck(mi, ctx, torch, dims, sc, xn, outs_n, 3)
            del keep_n

    # ---- CPU baseline: the oracle's ggml-cpu restatement of the same fc1 Q8_0 mul_mat
    # (from_float + vec_dot; AVX2, or AVX512-VNNI where the host has it), median of 5 after 2 warmups
    cpu = None
    if not args.no_cpu_baseline:
        log("bench: cpu baseline")
        wq = host_w[("q8_0", "fc1")]
        nth = orc.nthreads()
        xs_cpu = np.ascontiguousarray(x1024)
        times = []
        for i in range(7):
            t0 = time.perf_counter()
            orc.mul_mat(wq, orc.Q8_0, K, N, xs_cpu[None, None])
            if i >= 2:
                times.append(time.perf_counter() - t0)
        med = float(np.median(times))
        cpu_tops = 2.0 * M_TOK * N * K / med / 1e12
        cpu = {"value": round(cpu_tops, 4), "unit": "TOPS", "cores": nth, "kind": "port",
               "sample": f"fc1 Q8_0 mul_mat (quantize + block dots) 5184 x 4736 x 1024, median of 5 after 2 "
                         f"warmups: {med * 1e3:.1f} ms; {nth} threads (the host CPU share of one GPU) of "
                         f"nproc={os.cpu_count()}, isa={ISA_NAMES.get(orc.lib().orc_isa_path(), 'scalar')}, "
                         f"cpu={cpu_model()}"}

        if args.cpu_encoder_reps > 0 and not args.no_encoder:
            log("bench: cpu encoder baseline (one windowed + one global Q8_0 block)")
            cpu["vit_encoder_1008"] = cpu_encoder_baseline(orc, "q8_0", args.cpu_encoder_reps,
                                                           args.cpu_encoder_warmup)

    value = step_ops / (ms_step * 1e-3) / 1e12
    out = {
        "metric": "Q8_0/Q4_0 mul_mat TOPS (% MFMA peak); SAM3 ViT encoder ms/frame @1008²",
        "value": round(value, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: f32 N(0,0.02) weights quantized by ggml's reference quantizers, f32 N(0,1) activations, seed 0",
        "config": {"workload": "SAM3 ViT block linear set (qkv, proj, fc1, fc2) at 5184 tokens, Q8_0 and Q4_0 weights",
                   "tokens": M_TOK, "linears": [f"{n}x{k}" for (_, n, k) in LINEARS], "weight_types": TYPES},
        "pct_int8_peak": round(100.0 * value / INT8_PEAK_TOPS, 2),
        "weights": "prepared once at setup (mi355_weight_prepare, as a model load does); raw_layout_tops: "
                   "the same calls on ggml-layout weights, repacked on every call",
        "type_tops": {k: round(v, 2) for k, v in type_tops.items()},
        "raw_layout_tops": {k: round(v, 2) for k, v in raw_tops.items()},
        "config2_type_tops": cfg2,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "vit_encoder_1008": encoder,
        "hiera_tiny_1024": hiera,
        "sam3_neck_1008": neck_res,
        "attention": attn,
    }
    print(json.dumps(out), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
