"""ctypes loader for the plain-C oracle (oracle/_build/liboracle.so) — test infrastructure only."""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        lib = ctypes.CDLL(LIB)
        vp, i64 = ctypes.c_void_p, ctypes.c_int64
        lib.oracle_mxfp4_dequant.argtypes = [vp, vp, vp, i64, i64]
        lib.oracle_mxfp4_dequant.restype = None
        lib.oracle_mxfp4_linear.argtypes = [vp, i64, vp, vp, vp, i64, i64, ctypes.c_int]
        lib.oracle_mxfp4_linear.restype = None
        _lib = lib
    return _lib


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def mxfp4_dequant(codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    codes, scales = np.ascontiguousarray(codes, np.uint8), np.ascontiguousarray(scales, np.uint8)
    n, k = codes.shape[0], codes.shape[1] * 2
    out = np.empty((n, k), np.float32)
    load().oracle_mxfp4_dequant(_p(codes), _p(scales), _p(out), n, k)
    return out


def mxfp4_linear(x_bf16_bits: np.ndarray, codes: np.ndarray, scales: np.ndarray, nthreads: int = 1) -> np.ndarray:
    x = np.ascontiguousarray(x_bf16_bits, np.uint16)
    codes, scales = np.ascontiguousarray(codes, np.uint8), np.ascontiguousarray(scales, np.uint8)
    m, k = x.shape
    n = codes.shape[0]
    out = np.empty((m, n), np.float32)
    load().oracle_mxfp4_linear(_p(x), m, _p(codes), _p(scales), _p(out), n, k, int(nthreads))
    return out
