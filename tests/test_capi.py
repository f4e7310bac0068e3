"""The C-ABI library on the host: it loads, exports every entry point the
public header declares, and rejects invalid ggml operands with the right
status before touching the GPU (mirrors the failure modes sam3.cpp maps to
false at sam3.cpp:1023-1028)."""
import ctypes as C

import pytest


def test_exports_every_header_symbol(mi):
    L = mi.lib()
    syms = mi.header_symbols()
    assert len(syms) >= 12
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing


def test_abi_version(mi):
    """The header's MI355_ABI_VERSION is what the library reports."""
    import re
    with open(mi.HEADER) as f:
        want = int(re.search(r"#define MI355_ABI_VERSION (\d+)", f.read()).group(1))
    assert mi.lib().mi355_abi_version() == want == 2


def test_status_strings(mi):
    L = mi.lib()
    assert b"success" in L.mi355_status_to_string(0)
    assert b"not supported" in L.mi355_status_to_string(-3)


def mm(mi, t0=8, K=64, N=16, M=8, t1=0, tdst=0, ptr=0x1000):
    s0 = mi.make_tensor(ptr, t0, [K, N])
    s1 = mi.make_tensor(ptr, t1, [K, M])
    d = mi.make_tensor(ptr, tdst, [N, M])
    return s0, s1, d


def status(mi, s0, s1, d):
    return mi.lib().mi355_mul_mat(None, C.byref(s0), C.byref(s1), C.byref(d))


def test_mul_mat_validation(mi):
    L = mi.lib()
    s0, s1, d = mm(mi)
    assert L.mi355_supports_mul_mat(C.byref(s0), C.byref(s1), C.byref(d)) == 1
    assert status(mi, s0, s1, d) == -4  # valid operands, null context
    assert b"null context" in L.mi355_last_error(None)
    # K mismatch
    s0, s1, d = mm(mi)
    s1.ne[0] = 96
    assert status(mi, s0, s1, d) == -4
    # K not a multiple of the block size
    s0, s1, d = mm(mi, K=48)
    assert status(mi, s0, s1, d) == -4
    assert b"block size" in L.mi355_last_error(None)
    # unsupported dtypes
    assert status(mi, *mm(mi, t0=9)) == -3        # q8_1 weights
    assert status(mi, *mm(mi, t0=8, t1=1)) == -3  # f16 src1 with q8_0 src0
    assert status(mi, *mm(mi, tdst=1)) == -3      # f16 dst
    # broadcast ratio
    s0, s1, d = mm(mi)
    s0.ne[2] = 3
    s1.ne[2] = 4
    d.ne[2] = 4
    assert status(mi, s0, s1, d) == -4
    # null data pointer
    s0, s1, d = mm(mi)
    s1.data = None
    assert status(mi, s0, s1, d) == -4
    # non-contiguous src0 rows
    s0, s1, d = mm(mi)
    s0.nb[1] = 10
    assert status(mi, s0, s1, d) == -4
    # f16 rows of any K are taken (copied to a zero-padded pitch); odd addresses are not
    s0, s1, d = mm(mi, t0=1, K=12)
    assert mi.lib().mi355_supports_mul_mat(C.byref(s0), C.byref(s1), C.byref(d)) == 1
    s0.data = (s0.data or 0) + 1
    assert status(mi, s0, s1, d) == -4
    assert b"2-byte" in mi.lib().mi355_last_error(None)


def test_quantize_weights_validation(mi):
    L = mi.lib()
    src = mi.make_tensor(0x1000, 0, [64, 4])
    assert L.mi355_quantize_weights(None, 2, C.byref(src), C.c_void_p(0x2000)) == -4  # valid: null context
    assert b"null context" in L.mi355_last_error(None)
    assert L.mi355_quantize_weights(None, 9, C.byref(src), C.c_void_p(0x2000)) == -3  # q8_1 is an act type
    assert L.mi355_quantize_weights(None, 1, C.byref(src), C.c_void_p(0x2000)) == -3  # f16 is not a quant type
    src16 = mi.make_tensor(0x1000, 1, [64, 4])
    assert L.mi355_quantize_weights(None, 3, C.byref(src16), C.c_void_p(0x2000)) == -4  # f16 src accepted
    srcq = mi.make_tensor(0x1000, 8, [64, 4])
    assert L.mi355_quantize_weights(None, 2, C.byref(srcq), C.c_void_p(0x2000)) == -3  # quantized src
    src48 = mi.make_tensor(0x1000, 0, [48, 4])
    assert L.mi355_quantize_weights(None, 8, C.byref(src48), C.c_void_p(0x2000)) == -4
    assert b"block size" in L.mi355_last_error(None)
    assert L.mi355_quantize_weights(None, 8, C.byref(src), C.c_void_p(0x2001)) == -4  # odd dst
    assert L.mi355_model_quantize(None, b"a", b"b", 8, None) == -4


def test_quantize_rows_validation(mi):
    L = mi.lib()
    src = mi.make_tensor(0x1000, 0, [64, 4])
    assert L.mi355_quantize_rows(None, 8, 0, C.byref(src), C.c_void_p(0x2000)) == -4  # null context
    assert L.mi355_quantize_rows(None, 2, 0, C.byref(src), C.c_void_p(0x2000)) == -3  # q4_0 is not an act type
    assert L.mi355_quantize_rows(None, 8, 5, C.byref(src), C.c_void_p(0x2000)) == -4  # bad variant
    src = mi.make_tensor(0x1000, 0, [48, 4])
    assert L.mi355_quantize_rows(None, 8, 0, C.byref(src), C.c_void_p(0x2000)) == -4  # 48 % 32


def test_soft_max_and_fa_validation(mi):
    L = mi.lib()
    a = mi.make_tensor(0x1000, 0, [64, 4])
    b = mi.make_tensor(0x1000, 0, [64, 4])
    assert L.mi355_soft_max_ext(None, C.byref(a), C.byref(a), 1.0, 0.0, C.byref(b)) == -3  # mask unsupported
    assert L.mi355_soft_max_ext(None, C.byref(a), None, 1.0, 0.5, C.byref(b)) == -3       # ALiBi unsupported
    b.ne[1] = 5
    assert L.mi355_soft_max_ext(None, C.byref(a), None, 1.0, 0.0, C.byref(b)) == -4

    # flash_attn_ext: q [D, nq, nh, B], k/v [D, nkv, nhk, B], dst [D, nh, nq, B]
    def fa(D=64, nq=10, nkv=12, nh=4, nhk=2, tq=1, tk=1, tv=1, dne=None, vD=None):
        q = mi.make_tensor(0x1000, tq, [D, nq, nh, 1])
        k = mi.make_tensor(0x2000, tk, [D, nkv, nhk, 1])
        v = mi.make_tensor(0x3000, tv, [vD or D, nkv, nhk, 1])
        d = mi.make_tensor(0x4000, 0, dne or [vD or D, nh, nq, 1])
        return q, k, v, d

    def st(q, k, v, d, mask=None, bias=0.0, cap=0.0):
        return L.mi355_flash_attn_ext(None, C.byref(q), C.byref(k), C.byref(v), mask, 0.125, bias, cap, C.byref(d))

    q, k, v, d = fa()
    assert st(q, k, v, d) == -4                       # valid, null context
    assert b"null context" in L.mi355_last_error(None)
    assert st(q, k, v, d, mask=C.byref(q)) == -3      # mask unsupported
    assert st(q, k, v, d, bias=1.0) == -3             # ALiBi unsupported
    assert st(q, k, v, d, cap=50.0) == -3             # softcap unsupported
    assert st(*fa(D=80)) == -3                        # head size
    assert st(*fa(vD=128)) == -3                      # Dv != D: valid ggml, not implemented
    assert st(*fa(nhk=3)) == -4                       # 4 heads over 3 kv heads
    assert st(*fa(dne=[64, 10, 4, 1])) == -4          # dst must be [Dv, nh, nq, B]
    assert st(*fa(tk=1, tv=0)) == -3                  # k and v types differ
    assert st(*fa(tq=8)) == -3                        # quantized q


def test_workspace_size(mi):
    s0, s1, d = mm(mi, K=1024, N=4736, M=5184)
    n = mi.lib().mi355_mul_mat_workspace_size(C.byref(s0), C.byref(s1))
    assert n >= 5184 * 1024 + 5184 * 32 * 4
    # one activation row: the default (int8) route repacks the Q8_0 weights into the
    # workspace (N * K one-byte quants), far more than the fp16 route's operand needs
    s0, s1, d = mm(mi, K=1024, N=4736, M=1)
    assert mi.lib().mi355_mul_mat_workspace_size(C.byref(s0), C.byref(s1)) >= 4736 * 1024


def test_every_entry_point_rejects_null_arguments(mi):
    """Every entry point called with a NULL context / handle and null or zero
    arguments returns an error status (sizes return 0; the frees and the
    profile reset return) without touching a GPU, and a NULL-context failure
    leaves its text in mi355_last_error(NULL).  Run in a child process so that
    a crash fails the test instead of ending the session."""
    import subprocess, sys, textwrap
    code = textwrap.dedent(f"""
        import ctypes as C, importlib.util
        spec = importlib.util.spec_from_file_location("m", {mi.__file__!r})
        mi = importlib.util.module_from_spec(spec); spec.loader.exec_module(mi)
        L = mi.lib()
        # calls that create or query state without a context (or whose null arguments are valid)
        # are checked by their own tests: they may legitimately succeed
        skip = {{"mi355_context_create", "mi355_status_to_string", "mi355_last_error",
                 "mi355_model_file_last_error", "mi355_hiera_n_blocks", "mi355_buffer_alignment",
                 "mi355_abi_version"}}
        bad = []
        for name in sorted(mi.header_symbols()):
            if name in skip:
                continue
            fn = getattr(L, name)
            args = []
            for t in fn.argtypes:
                if t in (C.c_float, C.c_double):
                    args.append(0.0)
                elif t in (C.c_int, C.c_int32, C.c_int64, C.c_uint32, C.c_uint8, C.c_size_t):
                    args.append(0)
                else:
                    args.append(None)
            r = fn(*args)
            if fn.restype is None:
                continue
            if name.startswith("mi355_supports_"):
                if r != 0: bad.append((name, r))
            elif fn.restype == C.c_size_t:
                if r != 0: bad.append((name, r))
            elif fn.restype == C.c_int and name.endswith(("_find", "_hparams", "_collect")):
                if r > 0: bad.append((name, r))
            elif fn.restype == C.c_int:
                if r >= 0: bad.append((name, r))
                elif not L.mi355_last_error(None): bad.append((name, "no error text"))
        print("BAD", bad)
    """)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-3000:]
    assert "BAD []" in r.stdout, r.stdout


def fa_tensors(mi, D=64, n=40, nh=2, t=1, ptr=0x1000):
    q = mi.make_tensor(ptr, t, [D, n, nh, 1])
    k = mi.make_tensor(ptr, t, [D, n, nh, 1])
    v = mi.make_tensor(ptr, t, [D, n, nh, 1])
    o = mi.make_tensor(ptr, 0, [D, nh, n, 1])
    return q, k, v, o


def test_supports_flash_attn_and_soft_max(mi):
    """The supports queries (ggml_backend_supports_op per node kind) answer
    from the host checks of the entry points, with no context and no GPU."""
    L = mi.lib()
    q, k, v, o = fa_tensors(mi)
    assert L.mi355_supports_flash_attn_ext(q, k, v, None, 0.0, 0.0, o) == 1
    assert L.mi355_supports_flash_attn_ext(q, k, v, q, 0.0, 0.0, o) == 0      # a mask
    assert L.mi355_supports_flash_attn_ext(q, k, v, None, 1.0, 0.0, o) == 0   # ALiBi
    assert L.mi355_supports_flash_attn_ext(q, k, v, None, 0.0, 30.0, o) == 0  # softcap
    q2, k2, v2, o2 = fa_tensors(mi, D=80)
    assert L.mi355_supports_flash_attn_ext(q2, k2, v2, None, 0.0, 0.0, o2) == 0  # head size
    q3, k3, v3, o3 = fa_tensors(mi)
    o3.ne[1] = 3                                                               # dst shape
    assert L.mi355_supports_flash_attn_ext(q3, k3, v3, None, 0.0, 0.0, o3) == 0
    s = mi.make_tensor(0x1000, 0, [576, 576, 16, 1])
    d = mi.make_tensor(0x2000, 0, [576, 576, 16, 1])
    assert L.mi355_supports_soft_max_ext(s, None, 0.0, d) == 1
    assert L.mi355_supports_soft_max_ext(s, s, 0.0, d) == 0
    assert L.mi355_supports_soft_max_ext(s, None, 0.0, mi.make_tensor(0x2000, 1, [576, 576, 16, 1])) == 0
    assert L.mi355_supports_soft_max_ext(mi.make_tensor(0x1000, 0, [9000, 4]), None, 0.0,
                                         mi.make_tensor(0x2000, 0, [9000, 4])) == 0


def test_tensor_nbytes_is_ggml_nbytes(mi):
    L = mi.lib()
    assert L.mi355_tensor_nbytes(mi.make_tensor(0x1000, 8, [1024, 4736])) == 4736 * 32 * 34
    assert L.mi355_tensor_nbytes(mi.make_tensor(0x1000, 0, [64, 40, 2, 3])) == 64 * 40 * 2 * 3 * 4
    # a permuted view: the span from the first to one past the last element
    t = mi.make_tensor(0x1000, 0, [64, 40, 2, 1], nb=[4, 4 * 64 * 2, 4 * 64, 4 * 64 * 2 * 40])
    assert L.mi355_tensor_nbytes(t) == 4 + 63 * 4 + 39 * 4 * 64 * 2 + 1 * 4 * 64
    assert L.mi355_tensor_nbytes(mi.make_tensor(0x1000, 0, [64, 0])) == 0
    assert L.mi355_tensor_nbytes(mi.make_tensor(0x1000, 7, [64, 2], nb=[4, 256, 512, 512])) == 0  # unknown type


def test_prepared_weight_host_checks(mi):
    """Prepared-weight sizes and what MUL_MAT accepts as a prepared src0 (host
    side only: sizes, supports query)."""
    L = mi.lib()
    al = lambda v: (v + 255) // 256 * 256
    for t, N, K in [(8, 4736, 1024), (2, 1024, 4736), (3, 3072, 1024), (8, 7, 96), (3, 1, 32)]:
        dp = (K // 32 + 1) // 2 * 2
        want = al(N * K) + al(N * dp * 2) * (2 if t == 3 else 1)
        w = mi.make_tensor(0x1000, t, [K, N])
        assert L.mi355_weight_prepared_nbytes(C.byref(w)) == want
        pt = mi.make_tensor(0x1000, t, [K, N])
        pt.layout = mi.LAYOUT_INT8
        assert L.mi355_tensor_nbytes(C.byref(pt)) == want
    # not preparable: F16, 3-D, K not a multiple of 32, already prepared
    assert L.mi355_weight_prepared_nbytes(C.byref(mi.make_tensor(0x1000, 1, [64, 8]))) == 0
    assert L.mi355_weight_prepared_nbytes(C.byref(mi.make_tensor(0x1000, 8, [64, 8, 2]))) == 0
    w = mi.make_tensor(0x1000, 8, [64, 8])
    w.layout = mi.LAYOUT_INT8
    assert L.mi355_weight_prepared_nbytes(C.byref(w)) == 0
    t = mi.make_tensor(0x1000, 0, [64, 2])
    t.layout = 7  # unknown layout
    assert L.mi355_tensor_nbytes(C.byref(t)) == 0
    # MUL_MAT with a prepared src0: 2-D src1 only, 256-byte aligned data
    s0, s1, d = mm(mi)
    s0.layout = mi.LAYOUT_INT8
    s0.data = 0x10000
    assert L.mi355_supports_mul_mat(C.byref(s0), C.byref(s1), C.byref(d)) == 1
    s0.data = 0x10010
    assert L.mi355_supports_mul_mat(C.byref(s0), C.byref(s1), C.byref(d)) == 0
    s0.data = 0x10000
    s1.layout = mi.LAYOUT_INT8  # a prepared tensor is no src1
    assert L.mi355_supports_mul_mat(C.byref(s0), C.byref(s1), C.byref(d)) == 0
    assert status(mi, s0, s1, d) == -4


def test_buffer_api_host_checks(mi):
    L = mi.lib()
    assert L.mi355_buffer_alignment() == 256
    out = C.c_void_p()
    assert L.mi355_buffer_alloc(None, 1024, C.byref(out)) == -4 and not out.value
    assert L.mi355_buffer_place(None, 0, mi.make_tensor(0, 0, [4])) == -4
    t = mi.make_tensor(0x1000, 0, [16])
    buf = C.create_string_buffer(64)
    assert L.mi355_tensor_set(None, t, buf, 0, 64) == -4
    assert L.mi355_tensor_get(None, t, buf, 0, 64) == -4
    assert L.mi355_tensor_memset(None, t, 0, 0, 64) == -4
    assert L.mi355_buffer_base(None) is None and L.mi355_buffer_size(None) == 0
    L.mi355_buffer_free(None)  # no-op


def test_capi_program_without_gpu_fails_cleanly(mi):
    """The torch-free C++ caller (tests/native/capi_check) builds against the
    header; where no GPU is visible it reports that and exits with 2."""
    import os
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    subprocess.run(["make", "-s", "-C", os.path.join(root, "tests", "native")], check=True)
    r = subprocess.run([os.path.join(root, "tests", "native", "capi_check"),
                        os.path.join(root, "tests", "golden", "capi_fixture.bin")], capture_output=True, text=True,
                       timeout=120)
    if r.returncode == 0:  # a GPU is visible: the program ran its checks
        assert "capi_check ok" in r.stdout
    else:
        assert r.returncode == 2 and "mi355_context_create" in r.stderr, (r.returncode, r.stdout, r.stderr)


def test_supports_mul_mat_buffer_extents(mi):
    """The kernels address operands with 32-bit buffer offsets below 2^30 bytes: the
    supports query (host-only, dummy pointers) accepts the largest activation the
    int8 route holds (M * K just below 2^30 one-byte quants) and rejects one row
    more, for ggml-layout Q8_0 weights (whose fp16 route would need twice the
    bytes) and for a prepared weight; an F16 weight's fp16 route has half the room."""
    L = mi.lib()
    K, N = 4096, 64
    m_max = ((1 << 30) - 1) // K  # M * K < 2^30
    for t0, layout in ((8, 0), (8, 1), (2, 1)):
        for M, want in ((m_max, 1), (m_max + 1, 0)):
            s0, s1, d = mm(mi, t0=t0, K=K, N=N, M=M)
            if layout:
                s0.layout = mi.LAYOUT_INT8
                s0.nb[1] = K
                s0.nb[2] = s0.nb[3] = K * N
            assert L.mi355_supports_mul_mat(C.byref(s0), C.byref(s1), C.byref(d)) == want, (t0, layout, M)
    # F16 weights: ((M - 1) * K + K) * 2 < 2^30
    m_f16 = ((1 << 29) - 1) // K
    for M, want in ((m_f16, 1), (m_f16 + 1, 0)):
        s0, s1, d = mm(mi, t0=1, K=K, N=N, M=M)
        assert L.mi355_supports_mul_mat(C.byref(s0), C.byref(s1), C.byref(d)) == want, M
    s0, s1, d = mm(mi, t0=8, K=K, N=N, M=m_max + 1)
    assert status(mi, s0, s1, d) == -3
    assert b"extents" in L.mi355_last_error(None)
