"""Python host binding of libsam3mi355.so (the MI355X backend C-ABI of
include/sam3_mi355.h), used by the tests, bench.py and the smoke check.

The library is the product: every call here goes through its C entry
points.  If the shared library is missing this module raises instead of
falling back to anything else.  Device memory comes from torch tensors
(plumbing only); their data pointers are passed to the C-ABI.

The package directory is named ``sam3.cpp_amd``; load it with
``load_package()`` from a path, e.g.::

    spec = importlib.util.spec_from_file_location("sam3_cpp_amd", ".../sam3.cpp_amd/__init__.py")
"""
from __future__ import annotations

import ctypes as C
import os
import re
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "libsam3mi355.so")
HEADER = os.path.join(ROOT, "include", "sam3_mi355.h")

F32, F16, Q4_0, Q4_1, Q8_0, Q8_1 = 0, 1, 2, 3, 8, 9
ACT_X86, ACT_REF = 0, 1
MMQ_F16, MMQ_INT8, MMQ_AUTO = 0, 1, 2
LAYOUT_GGML, LAYOUT_INT8 = 0, 1
TYPE_SIZE = {F32: 4, F16: 2, Q4_0: 18, Q4_1: 20, Q8_0: 34, Q8_1: 36}
BLCK = {F32: 1, F16: 1, Q4_0: 32, Q4_1: 32, Q8_0: 32, Q8_1: 32}

STATUS = {-4: "INVALID_ARG", -3: "UNSUPPORTED", -2: "ALLOC_FAILED", -1: "FAILED", 0: "SUCCESS", 1: "ABORTED"}


class Mi355Error(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"{STATUS.get(status, status)}: {msg}")
        self.status = status


class Tensor(C.Structure):
    """struct mi355_tensor: the layout fields of a ggml_tensor."""
    _fields_ = [("type", C.c_int32), ("layout", C.c_int32), ("ne", C.c_int64 * 4),
                ("nb", C.c_int64 * 4), ("data", C.c_void_p)]


class VitHparams(C.Structure):
    """struct mi355_vit_hparams."""
    _fields_ = [("embed_dim", C.c_int32), ("num_heads", C.c_int32), ("mlp_dim", C.c_int32),
                ("window_size", C.c_int32), ("grid", C.c_int32), ("patch_size", C.c_int32),
                ("pos_grid", C.c_int32), ("eps", C.c_float)]


class VitBlock(C.Structure):
    """struct mi355_vit_block (device pointers)."""
    _fields_ = [("qkv_w", Tensor), ("proj_w", Tensor), ("fc1_w", Tensor), ("fc2_w", Tensor),
                ("norm1_w", C.c_void_p), ("norm1_b", C.c_void_p), ("qkv_b", C.c_void_p), ("proj_b", C.c_void_p),
                ("norm2_w", C.c_void_p), ("norm2_b", C.c_void_p), ("fc1_b", C.c_void_p), ("fc2_b", C.c_void_p),
                ("freqs_cis", C.c_void_p), ("is_global", C.c_int32)]


class HieraHparams(C.Structure):
    """struct mi355_hiera_hparams."""
    _fields_ = [("img_size", C.c_int32), ("embed_dim", C.c_int32), ("num_heads", C.c_int32),
                ("stages", C.c_int32 * 4), ("q_pool", C.c_int32), ("window_spec", C.c_int32 * 4),
                ("global_idx", C.c_int32 * 8), ("n_global", C.c_int32), ("eps", C.c_float)]


class HieraBlock(C.Structure):
    """struct mi355_hiera_block (device pointers)."""
    _fields_ = [("qkv_w", Tensor), ("proj_w", Tensor), ("fc1_w", Tensor), ("fc2_w", Tensor), ("dim_proj_w", Tensor),
                ("norm1_w", C.c_void_p), ("norm1_b", C.c_void_p), ("qkv_b", C.c_void_p), ("proj_b", C.c_void_p),
                ("norm2_w", C.c_void_p), ("norm2_b", C.c_void_p), ("fc1_b", C.c_void_p), ("fc2_b", C.c_void_p),
                ("dim_proj_b", C.c_void_p)]


class HieraBlockInfo(C.Structure):
    _fields_ = [("dim_in", C.c_int32), ("dim_out", C.c_int32), ("num_heads", C.c_int32),
                ("window_size", C.c_int32), ("q_stride", C.c_int32), ("stage", C.c_int32)]


def hiera_tiny(img_size: int = 1024) -> HieraHparams:
    """SAM2.1 Hiera-tiny (convert_sam2_to_ggml.py:81-84)."""
    hp = HieraHparams()
    hp.img_size, hp.embed_dim, hp.num_heads, hp.q_pool, hp.eps = img_size, 96, 1, 3, 1e-6
    for i, v in enumerate((1, 2, 7, 2)):
        hp.stages[i] = v
    for i, v in enumerate((8, 4, 14, 7)):
        hp.window_spec[i] = v
    for i, v in enumerate((5, 7, 9)):
        hp.global_idx[i] = v
    hp.n_global = 3
    return hp


def build(force: bool = False) -> str:
    """Compile the HIP sources for gfx950 (make -C sam3.cpp_amd)."""
    args = ["make", "-s", "-C", HERE, f"-j{min(16, os.cpu_count() or 1)}"]
    if force:
        subprocess.run(["make", "-s", "-C", HERE, "clean"], check=True)
    subprocess.run(args, check=True)
    return LIB_PATH


def header_symbols() -> list[str]:
    """Every function the public header declares."""
    with open(HEADER) as f:
        txt = f.read()
    return sorted(set(re.findall(r"^[A-Za-z_][\w\s\*]*?\b(mi355_\w+)\s*\(", txt, flags=re.M)))


_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build() (make -C sam3.cpp_amd)")
    L = C.CDLL(LIB_PATH)
    P, I, F, SZ = C.c_void_p, C.c_int, C.c_float, C.c_size_t
    T = C.POINTER(Tensor)
    sig = {
        "mi355_abi_version": (I, []),
        "mi355_context_create": (I, [I, P, C.POINTER(P)]),
        "mi355_context_free": (None, [P]),
        "mi355_synchronize": (I, [P]),
        "mi355_status_to_string": (C.c_char_p, [I]),
        "mi355_last_error": (C.c_char_p, [P]),
        "mi355_reserve_workspace": (I, [P, SZ]),
        "mi355_mul_mat_workspace_size": (SZ, [T, T]),
        "mi355_supports_mul_mat": (I, [T, T, T]),
        "mi355_buffer_alignment": (SZ, []),
        "mi355_buffer_alloc": (I, [P, SZ, C.POINTER(P)]),
        "mi355_buffer_free": (None, [P]),
        "mi355_buffer_base": (P, [P]),
        "mi355_buffer_size": (SZ, [P]),
        "mi355_buffer_place": (I, [P, SZ, T]),
        "mi355_buffer_clear": (I, [P, P, C.c_uint8]),
        "mi355_tensor_nbytes": (SZ, [T]),
        "mi355_tensor_set": (I, [P, T, P, SZ, SZ]),
        "mi355_tensor_get": (I, [P, T, P, SZ, SZ]),
        "mi355_tensor_memset": (I, [P, T, C.c_uint8, SZ, SZ]),
        "mi355_supports_flash_attn_ext": (I, [T, T, T, T, F, F, T]),
        "mi355_supports_soft_max_ext": (I, [T, T, F, T]),
        "mi355_mul_mat": (I, [P, T, T, T]),
        "mi355_mul_mat_noalloc": (I, [P, T, T, T]),
        "mi355_quantize_rows": (I, [P, I, I, T, P]),
        "mi355_quantize_weights": (I, [P, I, T, P]),
        "mi355_model_quantize": (I, [P, C.c_char_p, C.c_char_p, C.c_int32, C.POINTER(QuantizeStats)]),
        "mi355_mul_mat_block_dots": (I, [P, T, T, P]),
        "mi355_soft_max_ext": (I, [P, T, T, F, F, T]),
        "mi355_flash_attn_ext": (I, [P, T, T, T, T, F, F, F, T]),
        "mi355_vit_workspace_size": (SZ, [C.POINTER(VitHparams)]),
        "mi355_vit_prefix": (I, [P, C.POINTER(VitHparams), P, T, P, P, P, P]),
        "mi355_vit_block_forward": (I, [P, C.POINTER(VitHparams), C.POINTER(VitBlock), P]),
        "mi355_vit_encode": (I, [P, C.POINTER(VitHparams), P, T, P, P, P, C.POINTER(VitBlock), I, P]),
        "mi355_vit_layer_norm": (I, [P, P, P, I, P, P, P, C.c_int64, I, I, I, F]),
        "mi355_vit_qkv_rope": (I, [P, P, P, P, P, P, P, C.c_int64, I, I, I]),
        "mi355_vit_proj_residual": (I, [P, P, P, P, C.c_int64, I, I, I]),
        "mi355_vit_bias_gelu": (I, [P, P, P, C.c_int64, I]),
        "mi355_vit_bias_residual": (I, [P, P, P, P, C.c_int64, I]),
        "mi355_hiera_n_blocks": (I, [C.POINTER(HieraHparams)]),
        "mi355_hiera_block_info_get": (I, [C.POINTER(HieraHparams), I, C.POINTER(HieraBlockInfo)]),
        "mi355_hiera_workspace_size": (SZ, [C.POINTER(HieraHparams)]),
        "mi355_hiera_block_forward": (I, [P, C.POINTER(HieraHparams), I, C.POINTER(HieraBlock), P, I, P]),
        "mi355_hiera_prefix": (I, [P, C.POINTER(HieraHparams), P, T, P, P, P]),
        "mi355_hiera_encode": (I, [P, C.POINTER(HieraHparams), P, T, P, P, C.POINTER(HieraBlock), I,
                                   C.POINTER(P)]),
        "mi355_context_set_fusion": (I, [P, I]),
        "mi355_context_set_skinny": (I, [P, I]),
        "mi355_context_set_mmq_kernel": (I, [P, I]),
        "mi355_weight_prepared_nbytes": (SZ, [T]),
        "mi355_weight_prepare": (I, [P, T, P, SZ, T]),
        "mi355_hiera_pos_embed": (I, [P, P, I, I, I, P, I, I, I, P]),
        "mi355_neck_workspace_size": (SZ, [I, I, C.POINTER(NeckScale)]),
        "mi355_sam3_neck": (I, [P, P, I, I, C.POINTER(NeckScale), C.POINTER(P)]),
        "mi355_neck_deconv": (I, [P, T, P, P, I, I, I, P]),
        "mi355_neck_conv": (I, [P, T, P, P, I, I, P]),
        "mi355_neck_maxpool": (I, [P, P, I, I, I, P]),
        "mi355_model_file_open": (I, [C.c_char_p, C.POINTER(P)]),
        "mi355_model_file_close": (None, [P]),
        "mi355_model_file_last_error": (C.c_char_p, []),
        "mi355_model_file_header": (I, [P, C.POINTER(C.c_uint32), C.POINTER(I), C.POINTER(I), C.POINTER(I)]),
        "mi355_model_file_hparams": (I, [P, C.POINTER(C.POINTER(C.c_int32))]),
        "mi355_model_file_find": (I, [P, C.c_char_p]),
        "mi355_model_file_tensor": (I, [P, I, C.POINTER(ModelTensorInfo)]),
        "mi355_model_file_load_bytes": (SZ, [P, I, I]),
        "mi355_model_file_load": (I, [P, P, I, I, P, SZ]),
        "mi355_vit_weights_load": (I, [P, P, C.POINTER(P)]),
        "mi355_hiera_weights_load": (I, [P, P, C.POINTER(P)]),
        "mi355_hiera_weights_free": (None, [P]),
        "mi355_hiera_weights_get": (I, [P, C.POINTER(HieraHparams), C.POINTER(C.POINTER(HieraBlock)), C.POINTER(I),
                                        C.POINTER(C.POINTER(Tensor)), C.POINTER(P), C.POINTER(P)]),
        "mi355_vit_weights_free": (None, [P]),
        "mi355_vit_weights_get": (I, [P, C.POINTER(VitHparams), C.POINTER(C.POINTER(VitBlock)), C.POINTER(I),
                                      C.POINTER(C.POINTER(Tensor)), C.POINTER(P), C.POINTER(P), C.POINTER(P)]),
        "mi355_profile_enable": (I, [P, I]),
        "mi355_profile_collect": (I, [P]),
        "mi355_profile_get": (I, [P, I, C.POINTER(C.c_char_p), C.POINTER(I), C.POINTER(C.c_double)]),
        "mi355_profile_reset": (None, [P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


class NeckScale(C.Structure):
    """mi355_neck_scale: one SimpleFPN scale's kernels (mi355_tensor*) and biases."""
    _fields_ = [("deconv1_w", C.c_void_p), ("deconv1_b", C.c_void_p), ("deconv2_w", C.c_void_p),
                ("deconv2_b", C.c_void_p), ("conv1x1_w", C.c_void_p), ("conv1x1_b", C.c_void_p),
                ("conv3x3_w", C.c_void_p), ("conv3x3_b", C.c_void_p)]


class QuantizeStats(C.Structure):
    """mi355_quantize_stats: sam3_quantize_model's summary counts."""
    _fields_ = [("n_quantized", C.c_int32), ("n_total", C.c_int32), ("size_org", C.c_int64),
                ("size_new", C.c_int64)]


class ModelTensorInfo(C.Structure):
    _fields_ = [("name", C.c_char_p), ("type", C.c_int32), ("n_dims", C.c_int32), ("ne", C.c_int64 * 4),
                ("offset", C.c_uint64), ("nbytes", C.c_uint64)]


class ModelFile:
    """A sam3.cpp .ggml model file (header, hyperparameters, tensor index)."""

    def __init__(self, path: str):
        self.L = lib()
        self.h = C.c_void_p()
        st = self.L.mi355_model_file_open(os.fsencode(path), C.byref(self.h))
        if st != 0:
            raise Mi355Error(st, self.L.mi355_model_file_last_error().decode())

    def close(self):
        if self.h:
            self.L.mi355_model_file_close(self.h)
            self.h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def header(self):
        m, v, f, n = C.c_uint32(), C.c_int(), C.c_int(), C.c_int()
        st = self.L.mi355_model_file_header(self.h, C.byref(m), C.byref(v), C.byref(f), C.byref(n))
        if st != 0:
            raise Mi355Error(st, self.L.mi355_model_file_last_error().decode())
        return m.value, v.value, f.value, n.value

    def hparams(self) -> list:
        p = C.POINTER(C.c_int32)()
        n = self.L.mi355_model_file_hparams(self.h, C.byref(p))
        return [p[i] for i in range(n)]

    def find(self, name: str) -> int:
        return self.L.mi355_model_file_find(self.h, name.encode())

    def tensor(self, index: int) -> dict:
        info = ModelTensorInfo()
        st = self.L.mi355_model_file_tensor(self.h, index, C.byref(info))
        if st != 0:
            raise Mi355Error(st, self.L.mi355_model_file_last_error().decode())
        return {"name": info.name.decode(errors="replace"), "type": info.type, "n_dims": info.n_dims, "ne": list(info.ne),
                "offset": info.offset, "nbytes": info.nbytes}

    def load_bytes(self, index: int, dst_type: int) -> int:
        return self.L.mi355_model_file_load_bytes(self.h, index, dst_type)


def hiera_block_info(hp: HieraHparams, index: int) -> HieraBlockInfo:
    out = HieraBlockInfo()
    st = lib().mi355_hiera_block_info_get(C.byref(hp), index, C.byref(out))
    if st != 0:
        raise Mi355Error(st, lib().mi355_last_error(None).decode())
    return out


def row_size(t: int, ne0: int) -> int:
    return TYPE_SIZE[t] * (ne0 // BLCK[t])


def make_tensor(ptr: int, t: int, ne, nb=None) -> Tensor:
    """mi355_tensor over a device pointer, ggml ne (ne[0] contiguous); nb defaults to contiguous."""
    ne = list(ne) + [1] * (4 - len(ne))
    if nb is None:
        nb = [TYPE_SIZE[t], row_size(t, ne[0])]
        nb.append(nb[1] * ne[1])
        nb.append(nb[2] * ne[2])
    T = Tensor()
    T.type = t
    for i in range(4):
        T.ne[i] = int(ne[i])
        T.nb[i] = int(nb[i])
    T.data = ptr
    return T


def weight_prepared_nbytes(w: Tensor) -> int:
    """mi355_weight_prepared_nbytes."""
    return int(lib().mi355_weight_prepared_nbytes(C.byref(w)))


def from_torch(x, t: int, ne, nb=None) -> Tensor:
    """mi355_tensor viewing a torch tensor's storage (ggml ne order)."""
    T = make_tensor(x.data_ptr(), t, ne, nb)
    T._keep = x
    return T


class Context:
    """mi355_context on a device and stream (default: torch's current stream)."""

    def __init__(self, device: int = 0, stream: int | None = None):
        L = lib()
        if stream is None:
            import torch
            stream = torch.cuda.current_stream(device).cuda_stream
        h = C.c_void_p()
        st = L.mi355_context_create(device, C.c_void_p(stream), C.byref(h))
        if st != 0:
            raise Mi355Error(st, L.mi355_last_error(None).decode())
        self.h = h
        self.L = L

    def close(self):
        if self.h:
            self.L.mi355_context_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, st: int):
        if st != 0:
            raise Mi355Error(st, self.L.mi355_last_error(self.h).decode())

    def synchronize(self):
        self._check(self.L.mi355_synchronize(self.h))

    def mul_mat(self, src0: Tensor, src1: Tensor, dst: Tensor):
        self._check(self.L.mi355_mul_mat(self.h, C.byref(src0), C.byref(src1), C.byref(dst)))

    def mul_mat_noalloc(self, src0: Tensor, src1: Tensor, dst: Tensor):
        """mi355_mul_mat_noalloc: mi355_mul_mat with the library's fixed device scratch."""
        self._check(self.L.mi355_mul_mat_noalloc(self.h, C.byref(src0), C.byref(src1), C.byref(dst)))

    def mul_mat_block_dots(self, src0: Tensor, src1: Tensor, isums_ptr: int):
        self._check(self.L.mi355_mul_mat_block_dots(self.h, C.byref(src0), C.byref(src1), C.c_void_p(isums_ptr)))

    def quantize_rows(self, t: int, variant: int, src: Tensor, dst_ptr: int):
        self._check(self.L.mi355_quantize_rows(self.h, t, variant, C.byref(src), C.c_void_p(dst_ptr)))

    def hiera_pos_embed(self, bkg_ptr: int, E: int, bkg_h: int, bkg_w: int, win_ptr: int, ws: int, H: int, W: int,
                        out_ptr: int):
        self._check(self.L.mi355_hiera_pos_embed(self.h, C.c_void_p(bkg_ptr), E, bkg_h, bkg_w, C.c_void_p(win_ptr), ws,
                                                 H, W, C.c_void_p(out_ptr)))

    def neck_deconv(self, w: Tensor, b_ptr: int, x_ptr: int, H: int, W: int, gelu: bool, y_ptr: int):
        self._check(self.L.mi355_neck_deconv(self.h, C.byref(w), C.c_void_p(b_ptr), C.c_void_p(x_ptr), H, W,
                                             1 if gelu else 0, C.c_void_p(y_ptr)))

    def neck_conv(self, w: Tensor, b_ptr: int, x_ptr: int, H: int, W: int, y_ptr: int):
        self._check(self.L.mi355_neck_conv(self.h, C.byref(w), C.c_void_p(b_ptr), C.c_void_p(x_ptr), H, W,
                                           C.c_void_p(y_ptr)))

    def neck_maxpool(self, x_ptr: int, H: int, W: int, Cc: int, y_ptr: int):
        self._check(self.L.mi355_neck_maxpool(self.h, C.c_void_p(x_ptr), H, W, Cc, C.c_void_p(y_ptr)))

    def sam3_neck(self, x_ptr: int, E: int, G: int, scales, outs):
        """scales: 4 dicts of Tensor kernels / bias pointers; outs: 4 device pointers."""
        arr = (NeckScale * 4)()
        keep = []
        for i, s in enumerate(scales):
            for f in ("deconv1", "deconv2", "conv1x1", "conv3x3"):
                if s.get(f + "_w") is not None:
                    keep.append(s[f + "_w"])
                    setattr(arr[i], f + "_w", C.addressof(s[f + "_w"]))
                    setattr(arr[i], f + "_b", s[f + "_b"])
        o = (C.c_void_p * 4)(*outs)
        self._check(self.L.mi355_sam3_neck(self.h, C.c_void_p(x_ptr), E, G, arr, o))

    def quantize_weights(self, t: int, src: Tensor, dst_ptr: int):
        self._check(self.L.mi355_quantize_weights(self.h, t, C.byref(src), C.c_void_p(dst_ptr)))

    def model_quantize(self, in_path, out_path, qtype: int) -> QuantizeStats:
        """sam3_quantize_model: in_path -> out_path with qtype weights; returns the counts."""
        st = QuantizeStats()
        self._check(self.L.mi355_model_quantize(self.h, os.fsencode(str(in_path)), os.fsencode(str(out_path)), qtype,
                                                C.byref(st)))
        return st

    def soft_max_ext(self, src: Tensor, dst: Tensor, scale: float):
        self._check(self.L.mi355_soft_max_ext(self.h, C.byref(src), None, scale, 0.0, C.byref(dst)))

    def model_file_load(self, f: "ModelFile", index: int, dst_type: int, dst_ptr: int, dst_bytes: int):
        self._check(self.L.mi355_model_file_load(self.h, f.h, index, dst_type, C.c_void_p(dst_ptr), dst_bytes))

    def vit_weights_load(self, f: "ModelFile"):
        """(handle, hparams, blocks array, n, patch_w Tensor, pos, ln_w, ln_b) of the file's ViT."""
        w = C.c_void_p()
        self._check(self.L.mi355_vit_weights_load(self.h, f.h, C.byref(w)))
        hp = VitHparams()
        blocks = C.POINTER(VitBlock)()
        n = C.c_int()
        pw = C.POINTER(Tensor)()
        pos, lw, lb = C.c_void_p(), C.c_void_p(), C.c_void_p()
        self._check(self.L.mi355_vit_weights_get(w, C.byref(hp), C.byref(blocks), C.byref(n), C.byref(pw),
                                                 C.byref(pos), C.byref(lw), C.byref(lb)))
        return w, hp, blocks, n.value, pw.contents, pos.value, lw.value, lb.value

    def hiera_weights_load(self, f: "ModelFile"):
        """(handle, hparams, blocks array, n, patch_w Tensor, patch_b, pos) of the file's Hiera backbone."""
        w = C.c_void_p()
        self._check(self.L.mi355_hiera_weights_load(self.h, f.h, C.byref(w)))
        hp = HieraHparams()
        blocks = C.POINTER(HieraBlock)()
        n = C.c_int()
        pw = C.POINTER(Tensor)()
        pb, pos = C.c_void_p(), C.c_void_p()
        self._check(self.L.mi355_hiera_weights_get(w, C.byref(hp), C.byref(blocks), C.byref(n), C.byref(pw),
                                                   C.byref(pb), C.byref(pos)))
        return w, hp, blocks, n.value, pw.contents, pb.value, pos.value

    def hiera_weights_free(self, w):
        self.L.mi355_hiera_weights_free(w)

    def vit_weights_free(self, w):
        self.L.mi355_vit_weights_free(w)

    def set_fusion(self, enable: bool):
        """Encoder runners: producer passes write the MUL_MAT operand (default) or f32 rows."""
        self._check(self.L.mi355_context_set_fusion(self.h, 1 if enable else 0))

    def set_mmq_kernel(self, kernel: int):
        """Kernel of 2-D quantized MUL_MATs: MMQ_F16 (0), MMQ_INT8 (1) or MMQ_AUTO (2, the default); same bits."""
        self._check(self.L.mi355_context_set_mmq_kernel(self.h, int(kernel)))

    def weight_prepare(self, w: Tensor, dst: int, size: int) -> Tensor:
        """mi355_weight_prepare: w repacked into the device memory at dst (size bytes); the prepared tensor."""
        out = Tensor()
        self._check(self.L.mi355_weight_prepare(self.h, C.byref(w), C.c_void_p(dst), size, C.byref(out)))
        out._keep = getattr(w, "_keep", None)
        return out

    def set_mmq_int8(self, on: bool):
        self.set_mmq_kernel(MMQ_INT8 if on else MMQ_F16)

    def set_skinny(self, on: bool):
        self._check(self.L.mi355_context_set_skinny(self.h, 1 if on else 0))

    def profile(self, enable: bool):
        self._check(self.L.mi355_profile_enable(self.h, 1 if enable else 0))

    def profile_collect(self) -> dict:
        """{kernel name: (launches, total_ms)} of the launches timed so far; resets the totals."""
        n = self.L.mi355_profile_collect(self.h)
        if n < 0:
            self._check(n)
        out = {}
        for i in range(n):
            name, cnt, ms = C.c_char_p(), C.c_int(), C.c_double()
            self._check(self.L.mi355_profile_get(self.h, i, C.byref(name), C.byref(cnt), C.byref(ms)))
            out[name.value.decode()] = (cnt.value, ms.value)
        self.L.mi355_profile_reset(self.h)
        return out

    # ---- SAM3 ViT encoder (pointers are device addresses, e.g. tensor.data_ptr())
    def vit_layer_norm(self, x, add, add_grid, w, b, y, rows, E, grid=0, window=0, eps=1e-5):
        self._check(self.L.mi355_vit_layer_norm(self.h, x, add, add_grid, w, b, y, rows, E, grid, window, eps))

    def vit_qkv_rope(self, qkv, bias, rope, q, k, v, M, N, n_heads, head_dim):
        self._check(self.L.mi355_vit_qkv_rope(self.h, qkv, bias, rope, q, k, v, M, N, n_heads, head_dim))

    def vit_proj_residual(self, x, p, b, rows, E, grid=0, window=0):
        self._check(self.L.mi355_vit_proj_residual(self.h, x, p, b, rows, E, grid, window))

    def vit_bias_gelu(self, h, b, rows, n):
        self._check(self.L.mi355_vit_bias_gelu(self.h, h, b, rows, n))

    def vit_bias_residual(self, x, f, b, rows, n):
        self._check(self.L.mi355_vit_bias_residual(self.h, x, f, b, rows, n))

    def vit_prefix(self, hp: VitHparams, image, patch_w: Tensor, pos, ln_w, ln_b, x):
        self._check(self.L.mi355_vit_prefix(self.h, C.byref(hp), image, C.byref(patch_w), pos, ln_w, ln_b, x))

    def vit_block_forward(self, hp: VitHparams, blk: VitBlock, x):
        self._check(self.L.mi355_vit_block_forward(self.h, C.byref(hp), C.byref(blk), x))

    def vit_encode(self, hp: VitHparams, image, patch_w: Tensor, pos, ln_w, ln_b, blocks, x):
        arr = (VitBlock * len(blocks))(*blocks)
        self._check(self.L.mi355_vit_encode(self.h, C.byref(hp), image, C.byref(patch_w), pos, ln_w, ln_b, arr,
                                            len(blocks), x))

    # ---- SAM2 Hiera encoder
    def hiera_block_forward(self, hp: HieraHparams, index: int, blk: HieraBlock, x, spatial: int, x_out):
        self._check(self.L.mi355_hiera_block_forward(self.h, C.byref(hp), index, C.byref(blk), x, spatial, x_out))

    def hiera_prefix(self, hp: HieraHparams, image, patch_w: Tensor, patch_b, pos, x):
        self._check(self.L.mi355_hiera_prefix(self.h, C.byref(hp), image, C.byref(patch_w), patch_b, pos, x))

    def hiera_encode(self, hp: HieraHparams, image, patch_w: Tensor, patch_b, pos, blocks, stage_out=None):
        arr = (HieraBlock * len(blocks))(*blocks)
        outs = (C.c_void_p * 4)(*(stage_out or [None] * 4))
        self._check(self.L.mi355_hiera_encode(self.h, C.byref(hp), image, C.byref(patch_w), patch_b, pos, arr,
                                              len(blocks), outs))

    def flash_attn_ext(self, q: Tensor, k: Tensor, v: Tensor, dst: Tensor, scale: float):
        self._check(self.L.mi355_flash_attn_ext(self.h, C.byref(q), C.byref(k), C.byref(v), None, scale, 0.0, 0.0,
                                                C.byref(dst)))
