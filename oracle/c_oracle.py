"""ctypes wrapper over oracle/libnf4_oracle.so (the C restatement).

TEST INFRASTRUCTURE ONLY: used by tests/ as a second, independently written
restatement, and by bench.py's cpu_baseline leg as the timed CPU "port".
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libnf4_oracle.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.nf4o_quantize.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
        L.nf4o_quantize.restype = None
        L.nf4o_dequantize.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                                      ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
        L.nf4o_dequantize.restype = None
        L.nf4o_code.argtypes = [ctypes.c_float, ctypes.c_int]
        L.nf4o_code.restype = ctypes.c_int
        L.nf4o_check_cells.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                       ctypes.POINTER(ctypes.c_uint32)]
        L.nf4o_check_cells.restype = ctypes.c_int64
        _lib = L
    return _lib


_ROUND = {"argmin": 0, "threshold": 1}


def quantize(x: np.ndarray, dtype_tag: int, blocksize: int = 64, rounding: str = "argmin", threads: int = 0):
    x = np.ascontiguousarray(x)
    n = x.size
    packed = np.empty((n + 1) // 2, np.uint8)
    absmax = np.empty(-(-n // blocksize), np.float32)
    lib().nf4o_quantize(x.ctypes.data, dtype_tag, n, blocksize, _ROUND[rounding],
                        packed.ctypes.data, absmax.ctypes.data, threads)
    return packed, absmax


def dequantize(packed: np.ndarray, absmax: np.ndarray, n: int, blocksize: int, out_tag: int, threads: int = 0):
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    absmax = np.ascontiguousarray(absmax, dtype=np.float32)
    out = np.empty(n, np.float32 if out_tag == 2 else np.uint16)
    lib().nf4o_dequantize(packed.ctypes.data, absmax.ctypes.data, n, blocksize, out.ctypes.data, out_tag, threads)
    return out


def code(s: float, rounding: str) -> int:
    return lib().nf4o_code(ctypes.c_float(s), _ROUND[rounding])


def check_cells(bound: np.ndarray, base: np.ndarray, rounding: str):
    bound = np.ascontiguousarray(bound, np.float32)
    base = np.ascontiguousarray(base, np.uint8)
    first = ctypes.c_uint32(0)
    bad = lib().nf4o_check_cells(bound.ctypes.data, base.ctypes.data, bound.size, _ROUND[rounding],
                                 ctypes.byref(first))
    return int(bad), int(first.value)
