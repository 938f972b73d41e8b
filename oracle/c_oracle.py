"""ctypes binding of the plain-C oracle ``bfp8_ref.c`` (test infrastructure only)."""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle_bfp8.so")
_lib = None


def build():
    """Compile ``bfp8_ref.c`` with gcc (``oracle/Makefile``)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        p = ctypes.c_void_p
        i = ctypes.c_int
        _lib.oracle_quantize_bfp8.argtypes = [p, i, i, p, p]
        _lib.oracle_quantize_bfp8.restype = i
        _lib.oracle_quantize_bfp.argtypes = [p, i, i, p, p, i]
        _lib.oracle_quantize_bfp.restype = i
        _lib.oracle_dequantize_bfp8.argtypes = [p, p, i, i, p]
        _lib.oracle_swiglu_f32.argtypes = [p, p, p, p, p, p, p, i, i, i]
        _lib.oracle_f32_to_bf16_rne.argtypes = [ctypes.c_float]
        _lib.oracle_f32_to_bf16_rne.restype = ctypes.c_uint16
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def quantize(w_bits, mantissa_bits=7):
    w_bits = np.ascontiguousarray(w_bits, dtype=np.uint16)
    rows, cols = w_bits.shape
    q = np.zeros((rows, cols), np.int8)
    e8 = np.zeros((rows, cols // 16), np.uint8)
    bad = lib().oracle_quantize_bfp(_ptr(w_bits), rows, cols, _ptr(q), _ptr(e8), mantissa_bits)
    if bad:
        raise ValueError(f"{bad} groups hold non-finite values")
    return q, e8


def dequantize(q, e8):
    q = np.ascontiguousarray(q, dtype=np.int8)
    e8 = np.ascontiguousarray(e8, dtype=np.uint8)
    rows, cols = q.shape
    out = np.zeros((rows, cols), np.float32)
    lib().oracle_dequantize_bfp8(_ptr(q), _ptr(e8), rows, cols, _ptr(out))
    return out


def swiglu(x, wg, wu, wd, residual=None):
    x = np.ascontiguousarray(x, dtype=np.float32)
    wg = np.ascontiguousarray(wg, dtype=np.float32)
    wu = np.ascontiguousarray(wu, dtype=np.float32)
    wd = np.ascontiguousarray(wd, dtype=np.float32)
    M, H = x.shape
    I = wg.shape[0]
    hidden = np.zeros((M, I), np.float32)
    out = np.zeros((M, H), np.float32)
    res = None if residual is None else np.ascontiguousarray(residual, dtype=np.float32)
    lib().oracle_swiglu_f32(_ptr(x), _ptr(wg), _ptr(wu), _ptr(wd),
                            None if res is None else _ptr(res), _ptr(hidden), _ptr(out), M, H, I)
    return out


def f32_to_bf16_rne(value):
    return int(lib().oracle_f32_to_bf16_rne(float(value)))
