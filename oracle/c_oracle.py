"""ctypes binding of oracle/libsvq_oracle.so, the C restatement of the oracle.

TEST INFRASTRUCTURE ONLY: imported by tests/ and bench.py's CPU-baseline leg.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libsvq_oracle.so"
CODE = {"Q4_0": 4, "Q5_0": 5, "Q8_0": 8}
_lib = None


def build() -> Path:
    """Compile svq_oracle.c with gcc (make)."""
    subprocess.run(["make", "-s", "-C", str(HERE), "libsvq_oracle.so"], check=True)
    return LIB_PATH


def load():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(LIB_PATH))
        vp = ctypes.c_void_p
        lib.svqo_dequant.argtypes = [vp, vp, vp, ctypes.c_int64, ctypes.c_int]
        lib.svqo_dequant.restype = ctypes.c_int
        lib.svqo_gemv_f64.argtypes = [vp, vp, vp, vp, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_int, vp]
        lib.svqo_gemv_f64.restype = ctypes.c_int
        lib.svqo_half_to_float.argtypes = [ctypes.c_uint16]
        lib.svqo_half_to_float.restype = ctypes.c_float
        _lib = lib
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def dequant(q: np.ndarray, s: np.ndarray, qtype: str) -> np.ndarray:
    """Flat float32 weights of SoA arrays (q, s as uint8)."""
    q = np.ascontiguousarray(q, dtype=np.uint8)
    s = np.ascontiguousarray(s, dtype=np.uint8)
    nblocks = s.size // 2
    out = np.empty(nblocks * 32, dtype=np.float32)
    if load().svqo_dequant(_ptr(q), _ptr(s), _ptr(out), nblocks, CODE[qtype]) != 0:
        raise ValueError("svqo_dequant rejected its arguments")
    return out


def gemv_f64(x: np.ndarray, q: np.ndarray, s: np.ndarray, qtype: str, n: int, k: int,
             bias: np.ndarray | None = None) -> np.ndarray:
    """float64 [m, n] reference GEMV; x, bias as float16 arrays."""
    x = np.ascontiguousarray(x, dtype=np.float16)
    m = x.shape[0]
    q = np.ascontiguousarray(q, dtype=np.uint8)
    s = np.ascontiguousarray(s, dtype=np.uint8)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float16)
    y = np.empty((m, n), dtype=np.float64)
    rc = load().svqo_gemv_f64(_ptr(x), _ptr(q), _ptr(s), None if b is None else _ptr(b),
                              m, n, k, CODE[qtype], _ptr(y))
    if rc != 0:
        raise ValueError("svqo_gemv_f64 rejected its arguments")
    return y
