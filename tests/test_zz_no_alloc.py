"""mi355_mul_mat_noalloc, the MUL_MAT entry point that allocates nothing
(its scratch is the library's fixed per-GPU device array), against
mi355_mul_mat: same kernels and the same plan, so the results are equal bit
for bit.  Each weight type runs three calls in a row on the shared scratch,
each smaller than the one before (a split-K GEMM, a skinny K = 96 GEMM, a
small ragged one), so a later call must not read what an earlier call left;
and an operand set that needs more scratch than the array holds is
rejected on the host.  The K = 96 call reaches the int8 skinny kernel for
Q8_0 / Q4_0 (the int8 route under MI355_MMQ_AUTO), the fp16 route's skinny
kernel for Q4_1, and the tiled fp16 kernel for F16."""
import numpy as np
import pytest
import torch

from gpu_helpers import dev

pytestmark = pytest.mark.gpu

# (M, N, K): split-K (1024x1024 tiles over K = 4736), skinny (K = 96, M >= 4096), small ragged
CALLS = [(1024, 1024, 4736), (8192, 288, 96), (300, 200, 1024)]


def _weights(orc, t, N, K, seed):
    w = orc.normal(N * K, seed, 1, std=0.02).reshape(N, K)
    if t == orc.F16:
        return w.astype(np.float16).view(np.uint16)
    return orc.quantize_weights(t, w)


@pytest.mark.parametrize("tname", ["q8_0", "q4_0", "q4_1", "f16"])
def test_mul_mat_noalloc_matches_mul_mat(mi, ctx, orc, tname):
    t = orc.NAME_TYPE[tname]
    for i, (M, N, K) in enumerate(CALLS):
        print(f"noalloc {tname} call {i}: M={M} N={N} K={K}", flush=True)
        wq = _weights(orc, t, N, K, 300 + i)
        x = orc.normal(M * K, 301 + i, 2).reshape(M, K)
        wd, xd = dev(wq.view(np.uint8)), dev(x)
        s0 = mi.from_torch(wd, t, [K, N])
        s1 = mi.from_torch(xd, mi.F32, [K, M])
        ref = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        got = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        ctx.mul_mat(s0, s1, mi.from_torch(ref, mi.F32, [N, M]))
        ctx.mul_mat_noalloc(s0, s1, mi.from_torch(got, mi.F32, [N, M]))
        ctx.synchronize()
        assert torch.isfinite(ref).all()
        assert torch.equal(got, ref), f"call {i}: max diff {(got - ref).abs().max().item():.3e}"


def test_mul_mat_noalloc_rejects_oversized(mi, ctx, orc):
    M, N, K = 16384, 256, 4736  # the int8 operand alone: 16384 * 4736 one-byte quants = 77.6 MB > 64 MiB
    wq = _weights(orc, orc.Q8_0, N, K, 310)
    wd = dev(wq.view(np.uint8))
    xd = torch.zeros((M, K), dtype=torch.float32, device="cuda")
    out = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    s0, s1 = mi.from_torch(wd, mi.Q8_0, [K, N]), mi.from_torch(xd, mi.F32, [K, M])
    assert mi.lib().mi355_mul_mat_workspace_size(s0, s1) > (64 << 20)
    with pytest.raises(mi.Mi355Error) as ei:
        ctx.mul_mat_noalloc(s0, s1, mi.from_torch(out, mi.F32, [N, M]))
    assert ei.value.status == -3 and "scratch" in str(ei.value)
    ctx.synchronize()
    assert not out.any()


def test_mul_mat_noalloc_ordered_across_streams(mi, orc):
    """Two contexts on two streams share the GPU's one scratch array: each call
    waits on the event the other context's previous call recorded, so calls
    issued back to back with no host synchronization in between still give
    mi355_mul_mat's results (the first, a split-K GEMM, is the longest, so an
    unordered second call would overwrite its operand while it runs)."""
    s_a, s_b = torch.cuda.Stream(), torch.cuda.Stream()  # default priority
    ca, cb = mi.Context(0, s_a.cuda_stream), mi.Context(0, s_b.cuda_stream)
    try:
        shapes = [(1024, 1024, 4736), (2048, 512, 1024), (1024, 1024, 4736), (300, 200, 1024)]
        jobs = []
        for i, (M, N, K) in enumerate(shapes):
            wq = _weights(orc, orc.Q8_0, N, K, 320 + i)
            x = orc.normal(M * K, 321 + i, 2).reshape(M, K)
            wd, xd = dev(wq.view(np.uint8)), dev(x)
            s0, s1 = mi.from_torch(wd, mi.Q8_0, [K, N]), mi.from_torch(xd, mi.F32, [K, M])
            ref = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
            got = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
            jobs.append((s0, s1, ref, got, wd, xd))
        ctx_ref = mi.Context(0)
        try:
            for s0, s1, ref, got, _, _ in jobs:
                ctx_ref.mul_mat(s0, s1, mi.from_torch(ref, mi.F32, [ref.shape[1], ref.shape[0]]))
            ctx_ref.synchronize()
        finally:
            ctx_ref.close()
        torch.cuda.synchronize()
        for i, (s0, s1, ref, got, _, _) in enumerate(jobs):
            print(f"noalloc across streams: call {i} on context {'ab'[i % 2]}", flush=True)
            (ca if i % 2 == 0 else cb).mul_mat_noalloc(s0, s1, mi.from_torch(got, mi.F32, [got.shape[1], got.shape[0]]))
        ca.synchronize()
        cb.synchronize()
        for i, (_, _, ref, got, _, _) in enumerate(jobs):
            assert torch.isfinite(ref).all()
            assert torch.equal(got, ref), f"call {i}: max diff {(got - ref).abs().max().item():.3e}"
    finally:
        ca.close()
        cb.close()
