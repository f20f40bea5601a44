"""Builds the oracle's plain-C checker (codec.c) with gcc into oracle/_build/ — test
infrastructure, loaded only by tests through ``load()``."""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SOURCE = HERE / "codec.c"
OUT_DIR = HERE / "_build"
LIBRARY = OUT_DIR / "libmoe_oracle.so"


def build() -> Path:
    OUT_DIR.mkdir(exist_ok=True)
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-fno-fast-math", str(SOURCE), "-lm", "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode:
        raise RuntimeError(f"gcc failed:\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    return LIBRARY


_lib = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            build()
        lib = ctypes.CDLL(os.fspath(LIBRARY))
        P = ctypes.POINTER
        lib.oc_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        lib.oc_e4m3_to_f32.restype = ctypes.c_float
        lib.oc_f32_to_e4m3.argtypes = [ctypes.c_float]
        lib.oc_f32_to_e4m3.restype = ctypes.c_uint8
        lib.oc_f32_to_e4m3_array.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        lib.oc_f32_to_bf16.argtypes = [ctypes.c_float]
        lib.oc_f32_to_bf16.restype = ctypes.c_uint16
        lib.oc_f32_to_bf16_array.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        lib.oc_select.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                  ctypes.c_void_p]
        lib.oc_select.restype = ctypes.c_int
        lib.oc_permute.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                   ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        lib.oc_permute.restype = ctypes.c_int
        _lib = lib
    return _lib


def e4m3_encode(values) -> "object":
    """float32 numpy array -> uint8 codes."""
    import numpy as np

    x = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint8)
    load().oc_f32_to_e4m3_array(x.ctypes.data, out.ctypes.data, x.size)
    return out


def bf16_encode(values) -> "object":
    import numpy as np

    x = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    load().oc_f32_to_bf16_array(x.ctypes.data, out.ctypes.data, x.size)
    return out


def select(choice, K: int, G: int, top_groups: int):
    import numpy as np

    c = np.ascontiguousarray(choice, dtype=np.float32)
    ids = np.empty(K, dtype=np.int64)
    if load().oc_select(c.ctypes.data, c.size, K, G, top_groups, ids.ctypes.data):
        raise ValueError("oc_select: bad arguments")
    return ids


def permute(ids, E: int):
    import numpy as np

    a = np.ascontiguousarray(ids, dtype=np.int64)
    T, K = a.shape
    counts = np.empty(E, dtype=np.int32)
    offsets = np.empty(E + 1, dtype=np.int32)
    perm = np.empty(T * K, dtype=np.int32)
    inv = np.empty(T * K, dtype=np.int32)
    hit = load().oc_permute(a.ctypes.data, T, K, E, counts.ctypes.data, offsets.ctypes.data, perm.ctypes.data,
                            inv.ctypes.data)
    if hit < 0:
        raise ValueError("oc_permute: id out of range")
    return counts, offsets, perm, inv, hit
