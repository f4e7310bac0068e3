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
                 "mi355_model_file_last_error", "mi355_hiera_n_blocks", "mi355_supports_mul_mat"}}
        bad = []
        for name in sorted(mi.header_symbols()):
            if name in skip:
                continue
            fn = getattr(L, name)
            args = []
            for t in fn.argtypes:
                if t in (C.c_float, C.c_double):
                    args.append(0.0)
                elif t in (C.c_int, C.c_int32, C.c_int64, C.c_uint32, C.c_size_t):
                    args.append(0)
                else:
                    args.append(None)
            r = fn(*args)
            if fn.restype is None:
                continue
            if fn.restype == C.c_size_t:
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
