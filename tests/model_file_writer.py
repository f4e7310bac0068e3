"""Writes sam3.cpp .ggml model files for the loader tests.

Layout (the format sam3_load_model / sam3_load_tensors read, sam3.cpp:3095-3348):
little-endian u32 magic, i32 version, i32 ftype, i32 n_tensors; the
hyperparameters as i32 fields; then per tensor i32 n_dims, i32 name length,
i32 ggml type, i32 ne[0..n_dims) (ggml order), the name bytes, zero padding
to a 32-byte file offset, and the raw ggml rows.
"""
import struct

import numpy as np

MAGIC_SAM3, MAGIC_SAM2 = 0x73616D33, 0x73616D32


def sam3_hparams(img=1008, patch=14, embed=1024, depth=32, heads=16, mlp_x1000=4625, window=24,
                 global_idx=(7, 15, 23, 31), rest=None):
    """sam3_load_hparams field order (sam3.cpp:1481-1524); the 27 fields after
    the global-block list default to distinct small numbers."""
    h = [img, patch, embed, depth, heads, mlp_x1000, window, len(global_idx)]
    h += list(global_idx)[:4]
    h += list(rest) if rest is not None else [100 + i for i in range(27)]
    return h


def sam2_hparams(img=1024, backbone=1, rest=None):
    """sam2_load_hparams: img_size, backbone_type, then 55 more fields."""
    return [img, backbone] + (list(rest) if rest is not None else [200 + i for i in range(55)])


def write(path, magic, version, ftype, hparams, tensors, pad_byte=0, tail=b""):
    """tensors: list of (name, ggml type, ne tuple (ggml order), raw bytes);
    tail: bytes after the last tensor (where sam3.cpp files keep the tokenizer)."""
    with open(path, "wb") as f:
        f.write(struct.pack("<Iiii", magic, version, ftype, len(tensors)))
        f.write(struct.pack(f"<{len(hparams)}i", *hparams))
        for name, t, ne, data in tensors:
            nm = name.encode()
            f.write(struct.pack("<iii", len(ne), len(nm), t))
            f.write(struct.pack(f"<{len(ne)}i", *ne))
            f.write(nm)
            pos = f.tell()
            f.write(bytes([pad_byte]) * ((32 - pos % 32) % 32))
            f.write(np.ascontiguousarray(data).tobytes())
        f.write(tail)
