"""ctypes binding of oracle/int8_quant.c. TEST INFRASTRUCTURE ONLY."""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle_int8.so")
_lib = None


def build() -> str:
    """Compile the C oracle with oracle/Makefile; returns the library path."""
    subprocess.run(["make", "-s", "-C", _HERE, "_build/liboracle_int8.so"], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        lib.oracle_quantize_int8.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
        lib.oracle_quantize_int8.restype = ctypes.c_int
        lib.oracle_pack_tiles.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p]
        lib.oracle_pack_tiles.restype = ctypes.c_int
        lib.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        lib.oracle_f32_to_f16.restype = ctypes.c_uint16
        lib.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        lib.oracle_f16_to_f32.restype = ctypes.c_float
        _lib = lib
    return _lib


def quantize_per_channel(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    lib = _load()
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    q = np.empty((n, k), dtype=np.int8)
    s = np.empty((n,), dtype=np.uint16)
    rc = lib.oracle_quantize_int8(w.ctypes.data, n, k, q.ctypes.data, s.ctypes.data)
    if rc != 0:
        raise ValueError("weight contains non-finite values")
    return q, s.view(np.float16)


def pack_tiles(q: np.ndarray) -> np.ndarray:
    lib = _load()
    q = np.ascontiguousarray(q, dtype=np.int8)
    n, k = q.shape
    out = np.empty(n * k, dtype=np.uint8)
    if lib.oracle_pack_tiles(q.ctypes.data, n, k, out.ctypes.data) != 0:
        raise ValueError("bad shape for tile pack")
    return out


def f32_to_f16_bits(values: np.ndarray) -> np.ndarray:
    lib = _load()
    flat = np.asarray(values, dtype=np.float32).reshape(-1)
    return np.array([lib.oracle_f32_to_f16(float(v)) for v in flat], dtype=np.uint16)
