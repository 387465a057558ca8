"""ctypes binding of the C oracle (oracle/oracle.c -> oracle/_build/liboracle.so) -- TEST INFRASTRUCTURE ONLY."""

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_build", "liboracle.so")
_lib = None


def build():
    """Compile the C oracle with its Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        _lib = ctypes.CDLL(LIB)
        P, I64, INT = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        for name, args in {
            "oracle_quant_q8_0": [P, P, P, I64],
            "oracle_quant_q8_K": [P, P, P, P, I64],
            "oracle_block_dots": [INT, P, P, P, I64, I64, I64, I64],
            "oracle_reference_dot": [INT, P, P, P, P, I64, I64, I64],
            "oracle_gemv_f32": [INT, P, P, P, P, P, I64, I64, I64, I64],
            "oracle_quantize_q4_0": [P, P, I64],
        }.items():
            getattr(_lib, name).argtypes = args
            getattr(_lib, name).restype = None
        _lib.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        _lib.oracle_f32_to_f16.restype = ctypes.c_uint16
        _lib.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        _lib.oracle_f16_to_f32.restype = ctypes.c_float
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def quant_q8_0(x):
    x = np.ascontiguousarray(x, np.float32)
    m, k = x.shape
    q = np.empty((m, k), np.int8)
    d = np.empty((m, k // 32), np.float32)
    lib().oracle_quant_q8_0(_p(x), _p(q), _p(d), m * (k // 32))
    return q, d


def quant_q8_K(x):
    x = np.ascontiguousarray(x, np.float32)
    m, k = x.shape
    q = np.empty((m, k), np.int8)
    d = np.empty((m, k // 256), np.float32)
    bs = np.empty((m, k // 16), np.int16)
    lib().oracle_quant_q8_K(_p(x), _p(q), _p(d), _p(bs), m * (k // 256))
    return q, d, bs


FMT = {"q4_0": 0, "tq2_0": 1}


def block_dots(fmt, wq, xq, n, k):
    wq = np.ascontiguousarray(wq, np.uint8)
    xq = np.ascontiguousarray(xq, np.int8)
    m = xq.shape[0]
    nb = k // (32 if fmt == "q4_0" else 256)
    s = np.empty((m, n, nb), np.int64)
    lib().oracle_block_dots(FMT[fmt], _p(wq), _p(xq), _p(s), m, n, k, wq.shape[1])
    return s


def reference_dot(fmt, ws, xd, s):
    ws = np.ascontiguousarray(ws, np.int16)
    xd = np.ascontiguousarray(xd, np.float32)
    s = np.ascontiguousarray(s, np.int64)
    m, n, nb = s.shape
    r = np.empty((m, n), np.float64)
    lib().oracle_reference_dot(FMT[fmt], _p(ws), _p(xd), _p(s), _p(r), m, n, nb)
    return r


def gemv_f32(fmt, wq, ws, xq, xd, n, k):
    wq = np.ascontiguousarray(wq, np.uint8)
    ws = np.ascontiguousarray(ws, np.int16)
    xq = np.ascontiguousarray(xq, np.int8)
    xd = np.ascontiguousarray(xd, np.float32)
    m = xq.shape[0]
    y = np.empty((m, n), np.float32)
    lib().oracle_gemv_f32(FMT[fmt], _p(wq), _p(ws), _p(xq), _p(xd), _p(y), m, n, k, wq.shape[1])
    return y


def quantize_q4_0_weights(w):
    """f32 [n][k] -> ggml q4_0 blocks (bytes), as oracle.quantize_q4_0_weights."""
    w = np.ascontiguousarray(w, np.float32)
    n, k = w.shape
    out = np.empty(n * (k // 32) * 18, np.uint8)
    lib().oracle_quantize_q4_0(_p(w), _p(out), n * (k // 32))
    return out.tobytes()
