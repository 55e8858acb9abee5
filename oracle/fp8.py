"""TEST INFRASTRUCTURE ONLY: ctypes binding of the C E4M3FN codec oracle.

The codec restates flash_attn_mps/kernels/cache.metal:8-18 (encode) and
flash_attn_mps/kernels/attention.metal:4-10 (decode); see fp8_e4m3.c.
"""
import ctypes
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "liboracle_fp8.so"
_lib = None


def build():
    subprocess.run(["make", "-C", str(_HERE), "-B"], check=True,
                   stdout=subprocess.DEVNULL)


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(_LIB_PATH))
        f32p = ctypes.POINTER(ctypes.c_float)
        u8p = ctypes.POINTER(ctypes.c_uint8)
        _lib.oracle_e4m3_encode_array.argtypes = [f32p, u8p, ctypes.c_int64]
        _lib.oracle_e4m3_decode_array.argtypes = [u8p, f32p, ctypes.c_int64]
        _lib.oracle_e4m3_encode_scaled.argtypes = [f32p, f32p, ctypes.c_int64, ctypes.c_int64,
                                                   ctypes.c_int64, ctypes.c_int64, u8p]
        _lib.oracle_e4m3_sweep.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int64, u8p]
        _lib.oracle_e4m3_sweep.restype = ctypes.c_int64
    return _lib


def _ptr(a, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def encode(values):
    """float32 array -> uint8 E4M3FN codes (same shape)."""
    x = np.ascontiguousarray(np.asarray(values, dtype=np.float32))
    out = np.empty(x.shape, dtype=np.uint8)
    lib().oracle_e4m3_encode_array(_ptr(x, ctypes.c_float), _ptr(out, ctypes.c_uint8), x.size)
    return out


def encode_scaled(x, scale):
    """x [rows, heads, dim] float32, scale [1] or [heads] -> codes of x / scale[h]."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    s = np.ascontiguousarray(np.asarray(scale, dtype=np.float32).reshape(-1))
    rows, heads, dim = x.shape
    out = np.empty(x.shape, dtype=np.uint8)
    lib().oracle_e4m3_encode_scaled(_ptr(x, ctypes.c_float), _ptr(s, ctypes.c_float), rows, heads, dim,
                                    0 if s.size == 1 else 1, _ptr(out, ctypes.c_uint8))
    return out


def decode(codes):
    """uint8 E4M3FN codes -> float32 values."""
    b = np.ascontiguousarray(np.asarray(codes, dtype=np.uint8))
    out = np.empty(b.shape, dtype=np.float32)
    lib().oracle_e4m3_decode_array(_ptr(b, ctypes.c_uint8), _ptr(out, ctypes.c_float), b.size)
    return out


def sweep(start, stride, count):
    """Encode the floats with bit patterns start + k*stride, k < count."""
    out = np.empty(count, dtype=np.uint8)
    lib().oracle_e4m3_sweep(start, stride, count, _ptr(out, ctypes.c_uint8))
    return out
