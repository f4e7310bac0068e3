"""The C-ABI driven without torch or Python: tests/native/capi_check (C++,
include/sam3_mi355.h only) allocates device buffers through the buffer API,
uploads the committed fixture tests/golden/capi_fixture.bin, runs a Q8_0
MUL_MAT and a FLASH_ATTN_EXT and checks them against the oracle results the
fixture holds (1e-5 * absterm and 2e-3 * attention of |V|).  Also the buffer
API through ctypes: set/get round trips, memsets of unaligned ranges (the
fill kernel's head, 16-byte body and tail), clears and bounds."""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_capi_program():
    exe = os.path.join(ROOT, "tests", "native", "capi_check")
    assert os.path.exists(exe), "build tests/native first (__graft_entry__.build())"
    print("running tests/native/capi_check", flush=True)
    r = subprocess.run([exe, os.path.join(ROOT, "tests", "golden", "capi_fixture.bin")], capture_output=True,
                       text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0 and "capi_check ok" in r.stdout, (r.returncode, r.stdout, r.stderr)


def test_buffer_api(mi, ctx):
    L = mi.lib()
    buf = C.c_void_p()
    ctx._check(L.mi355_buffer_alloc(ctx.h, 1 << 20, C.byref(buf)))
    try:
        assert L.mi355_buffer_size(buf) == 1 << 20 and L.mi355_buffer_base(buf) % 256 == 0
        t = mi.make_tensor(0, mi.F32, [1000, 7])  # 28000 bytes
        assert L.mi355_buffer_place(buf, 100, t) == -4          # unaligned offset
        assert L.mi355_buffer_place(buf, (1 << 20) - 256, t) == -4  # does not fit
        ctx._check(L.mi355_buffer_place(buf, 512, t))
        assert t.data == L.mi355_buffer_base(buf) + 512
        ctx._check(L.mi355_buffer_clear(ctx.h, buf, 0x5A))
        rng = np.random.default_rng(1)
        src = rng.standard_normal(7000).astype(np.float32)
        ctx._check(L.mi355_tensor_set(ctx.h, t, src.ctypes.data, 0, src.nbytes))
        back = np.empty_like(src)
        ctx._check(L.mi355_tensor_get(ctx.h, t, back.ctypes.data, 0, back.nbytes))
        assert np.array_equal(back, src)
        ref = src.view(np.uint8).copy()
        for off, n, val in [(0, 1, 1), (3, 13, 2), (5, 16, 3), (17, 1000, 4), (16, 32, 5), (27000, 1000, 6),
                            (1, 27999, 7)]:
            ctx._check(L.mi355_tensor_memset(ctx.h, t, val, off, n))
            ref[off:off + n] = val
            got = np.empty(28000, dtype=np.uint8)
            ctx._check(L.mi355_tensor_get(ctx.h, t, got.ctypes.data, 0, 28000))
            assert np.array_equal(got, ref), (off, n, val)
        # the bytes around the tensor keep the clear value
        pre = mi.make_tensor(L.mi355_buffer_base(buf), mi.F32, [128])
        got = np.empty(512, dtype=np.uint8)
        ctx._check(L.mi355_tensor_get(ctx.h, pre, got.ctypes.data, 0, 512))
        assert (got == 0x5A).all()
        assert L.mi355_tensor_set(ctx.h, t, src.ctypes.data, 4, src.nbytes) == -4  # past the end
        assert L.mi355_tensor_memset(ctx.h, t, 0, 27999, 2) == -4
    finally:
        L.mi355_buffer_free(buf)
