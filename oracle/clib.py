"""ctypes binding of ``oracle/liboracle.so`` (test infrastructure only; see package header)."""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / "liboracle.so"
_LIB = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIBRARY


def lib():
    global _LIB
    if _LIB is None:
        if not LIBRARY.exists():
            build()
        handle = ctypes.CDLL(str(LIBRARY))
        p = ctypes.c_void_p
        i64 = ctypes.c_int64
        handle.oracle_palette.argtypes = [p]
        handle.oracle_decode_bf16.argtypes = [p, p, i64, i64, p, p]
        handle.oracle_matvec_f64.argtypes = [p, p, i64, i64, p]
        handle.oracle_gemm_f64.argtypes = [p, p, i64, i64, i64, p]
        handle.oracle_decode_matvec_f32.argtypes = [p, p, p, i64, i64, p]
        handle.oracle_max_threads.restype = ctypes.c_int
        handle.oracle_set_threads.argtypes = [ctypes.c_int]
        _LIB = handle
    return _LIB


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def palette() -> np.ndarray:
    out = np.empty((255, 255, 8), dtype=np.float32)
    lib().oracle_palette(_ptr(out))
    return out


def decode_bf16_bits(blocks: np.ndarray, scales: np.ndarray, lut: np.ndarray | None = None) -> np.ndarray:
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    m = scales.shape[0]
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(m, -1)
    bpr = blocks.shape[1] // 8
    out = np.empty((m, bpr * 16), dtype=np.uint16)
    lut_ptr = None
    if lut is not None:
        lut = np.ascontiguousarray(lut, dtype=np.float32)
        lut_ptr = _ptr(lut)
    lib().oracle_decode_bf16(_ptr(blocks), _ptr(scales), m, bpr, lut_ptr, _ptr(out))
    return out


def matvec_f64(w_bits: np.ndarray, x_bits: np.ndarray) -> np.ndarray:
    w_bits = np.ascontiguousarray(w_bits, dtype=np.uint16)
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16).reshape(-1)
    m, k = w_bits.shape
    y = np.empty(m, dtype=np.float64)
    lib().oracle_matvec_f64(_ptr(w_bits), _ptr(x_bits), m, k, _ptr(y))
    return y


def gemm_f64(x_bits: np.ndarray, w_bits: np.ndarray) -> np.ndarray:
    w_bits = np.ascontiguousarray(w_bits, dtype=np.uint16)
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    t, k = x_bits.shape
    m = w_bits.shape[0]
    y = np.empty((t, m), dtype=np.float64)
    lib().oracle_gemm_f64(_ptr(x_bits), _ptr(w_bits), t, m, k, _ptr(y))
    return y


def decode_matvec_f32(blocks: np.ndarray, scales: np.ndarray, x_bits: np.ndarray) -> np.ndarray:
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    m = scales.shape[0]
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(m, -1)
    bpr = blocks.shape[1] // 8
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16).reshape(-1)
    y = np.empty(m, dtype=np.float32)
    lib().oracle_decode_matvec_f32(_ptr(blocks), _ptr(scales), _ptr(x_bits), m, bpr, _ptr(y))
    return y


def set_threads(n: int) -> None:
    lib().oracle_set_threads(int(n))


def max_threads() -> int:
    return int(lib().oracle_max_threads())
