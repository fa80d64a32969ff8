"""Locates and loads the in-tree native libraries of this package.

Both libraries are built in place by `make -C ziggy-llm_amd` (or
__graft_entry__.build()).  A missing library is an error: there is no
fallback path.
"""
from __future__ import annotations

import ctypes
import os

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD_DIR = os.path.join(PKG_DIR, "build")
HIP_LIB = os.path.join(BUILD_DIR, "libziggy_hip.so")
SYNTH_LIB = os.path.join(BUILD_DIR, "libziggy_synth.so")

_cache: dict = {}


def load(path: str) -> ctypes.CDLL:
    if path in _cache:
        return _cache[path]
    if not os.path.exists(path):
        raise RuntimeError(f"{os.path.basename(path)} is not built ({path}); run `make -C {PKG_DIR}` first")
    lib = ctypes.CDLL(path)
    _cache[path] = lib
    return lib


def synth() -> ctypes.CDLL:
    lib = load(SYNTH_LIB)
    if not getattr(lib, "_zs_typed", False):
        u8p = ctypes.c_void_p
        lib.zs_fill_tensor.argtypes = [u8p, ctypes.c_int, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64,
                                       ctypes.c_float, ctypes.c_float, ctypes.c_int]
        lib.zs_fill_tensor.restype = ctypes.c_int
        lib.zs_quantize_row.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p]
        lib.zs_quantize_row.restype = ctypes.c_int
        lib.zs_normal_row.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_float, ctypes.c_float,
                                      ctypes.c_void_p, ctypes.c_uint64]
        lib.zs_normal_row.restype = None
        lib._zs_typed = True
    return lib
