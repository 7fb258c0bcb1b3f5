"""ctypes binding of the C oracle (``oracle/libqmm_oracle.so``).  TEST INFRASTRUCTURE ONLY."""

from __future__ import annotations

import ctypes
import os

import numpy as np

from .build import OUT

_lib = None
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int

DTYPE_CODE = {"bfloat16": 0, "float16": 1}


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(OUT):
            from .build import build
            build()
        h = ctypes.CDLL(OUT)
        h.oracle_dequantize.restype = _int
        h.oracle_dequantize.argtypes = [_vp, _vp, _vp, _vp, _i64, _i64, _int, _int, _int]
        h.oracle_qmm.restype = _int
        h.oracle_qmm.argtypes = [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _int, _int, _int]
        h.oracle_gather_qmm.restype = _int
        h.oracle_gather_qmm.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                                        _i64, _i64, _int, _int, _int, _int]
        h.oracle_round_bf16.restype = ctypes.c_uint16
        h.oracle_round_bf16.argtypes = [ctypes.c_float]
        h.oracle_round_f16.restype = ctypes.c_uint16
        h.oracle_round_f16.argtypes = [ctypes.c_float]
        _lib = h
    return _lib


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def dequantize(w, s, b, group_size, bits, dtype="bfloat16") -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint32)
    s = np.ascontiguousarray(s, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    N = w.shape[0]
    K = w.shape[1] * 32 // bits
    out = np.empty((N, K), dtype=np.uint16)
    rc = lib().oracle_dequantize(_p(w), _p(s), _p(b), _p(out), N, K, group_size, bits,
                                 DTYPE_CODE[dtype])
    if rc:
        raise ValueError(f"oracle_dequantize rc={rc}")
    return out


def qmm(x, w, s, b, group_size, bits, dtype="bfloat16", threads=0) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint32)
    s = np.ascontiguousarray(s, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    M, K = x.shape
    N = w.shape[0]
    out = np.empty((M, N), dtype=np.float32)
    rc = lib().oracle_qmm(_p(x), _p(w), _p(s), _p(b), _p(out), M, N, K, group_size, bits,
                          DTYPE_CODE[dtype], threads)
    if rc:
        raise ValueError(f"oracle_qmm rc={rc}")
    return out


def gather_qmm(x, w, s, b, lhs, rhs, group_size, bits, dtype="bfloat16", threads=0) -> np.ndarray:
    """x [B, M, K], w [E, N, Kw] -> out [P, M, N] float32 (C oracle's per-pair loop)."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint32)
    s = np.ascontiguousarray(s, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    lhs = np.ascontiguousarray(lhs, dtype=np.int32)
    rhs = np.ascontiguousarray(rhs, dtype=np.int32)
    B, M, K = x.shape
    E, N = w.shape[0], w.shape[1]
    P = rhs.shape[0]
    out = np.empty((P, M, N), dtype=np.float32)
    rc = lib().oracle_gather_qmm(_p(x), _p(w), _p(s), _p(b), _p(lhs), _p(rhs), _p(out), P, M, N,
                                 K, E, B, group_size, bits, DTYPE_CODE[dtype], threads)
    if rc:
        raise ValueError(f"oracle_gather_qmm rc={rc}")
    return out
