"""ctypes binding of ``libmlxturbo_amd.so`` (C ABI in ``include/mlxturbo_amd.h``).

The library is built in-tree by :mod:`mlxturbo_amd.build`.  There is no
fallback: if the library is missing every operator raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

LIB_NAME = "libmlxturbo_amd.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

MQ_OK = 0
MQ_EINVAL = -1
MQ_EUNSUPPORTED = -2

MQ_BFLOAT16 = 0
MQ_FLOAT16 = 1
MQ_FLOAT32 = 2

# every symbol include/mlxturbo_amd.h declares
EXPORTED = (
    "mq_version",
    "mq_last_error",
    "mq_launch_count",
    "mq_set_row_identity",
    "mq_dequantize",
    "mq_quantize",
    "mq_quantized_matmul",
    "mq_quantized_matmul_workspace_size",
    "mq_quantized_matmul_ws",
    "mq_gather_qmm_workspace_size",
    "mq_gather_qmm",
    "mq_gather_qmm_noalloc",
    "mq_gather_tables",
    "mq_gather_qmm_tables",
    "mq_gather_swiglu_tables",
    "mq_swiglu",
    "mq_moe_glu_route",
    "mq_moe_block",
    "mq_moe_layer",
    "mq_gather_glu",
    "mq_gather_qmm_combine",
    "mq_moe_combine",
    "mq_moe_combine_shared",
    "mq_moe_route",
)

_lock = threading.Lock()
_lib = None

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_sz = ctypes.c_size_t


class LibraryMissing(RuntimeError):
    pass


def _bind(lib: ctypes.CDLL) -> None:
    lib.mq_version.restype = _int
    lib.mq_version.argtypes = []
    lib.mq_last_error.restype = ctypes.c_char_p
    lib.mq_last_error.argtypes = []
    lib.mq_launch_count.restype = ctypes.c_uint64
    lib.mq_launch_count.argtypes = []
    lib.mq_set_row_identity.restype = _int
    lib.mq_set_row_identity.argtypes = [_int]
    lib.mq_dequantize.restype = _int
    lib.mq_dequantize.argtypes = [_vp, _vp, _vp, _vp, _i64, _i64, _int, _int, _int, _vp]
    lib.mq_quantize.restype = _int
    lib.mq_quantize.argtypes = [_vp, _vp, _vp, _vp, _i64, _i64, _int, _int, _int, _vp]
    lib.mq_quantized_matmul.restype = _int
    lib.mq_quantized_matmul.argtypes = [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _int,
                                        _int, _int, _vp]
    lib.mq_quantized_matmul_workspace_size.restype = ctypes.c_size_t
    lib.mq_quantized_matmul_workspace_size.argtypes = [_i64, _i64, _i64, _int, _int]
    lib.mq_quantized_matmul_ws.restype = _int
    lib.mq_quantized_matmul_ws.argtypes = [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _int,
                                           _int, _int, _vp, ctypes.c_size_t, _vp]
    lib.mq_gather_qmm_workspace_size.restype = ctypes.c_size_t
    lib.mq_gather_qmm_workspace_size.argtypes = [_i64, _i64]
    lib.mq_gather_qmm.restype = _int
    lib.mq_gather_qmm.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                                  _i64, _i64, _int, _int, _int, _int, _vp, ctypes.c_size_t, _vp]
    lib.mq_gather_qmm_noalloc.restype = _int
    lib.mq_gather_qmm_noalloc.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64,
                                          _i64, _i64, _i64, _int, _int, _int, _int, _vp]
    lib.mq_gather_tables.restype = _int
    lib.mq_gather_tables.argtypes = [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _sz, _vp]
    lib.mq_gather_qmm_tables.restype = _int
    lib.mq_gather_qmm_tables.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64,
                                         _i64, _i64, _i64, _int, _int, _int, _vp, _sz, _vp]
    lib.mq_gather_swiglu_tables.restype = _int
    lib.mq_gather_swiglu_tables.argtypes = [_vp] * 10 + [_i64] * 6 + [_int, _int, _int, _vp,
                                                                      _sz, _vp]
    lib.mq_moe_glu_route.restype = _int
    lib.mq_moe_glu_route.argtypes = [_vp] * 13 + [_i64] * 5 + [_int, _int, _int, _vp]
    lib.mq_moe_block.restype = _int
    lib.mq_moe_block.argtypes = [_vp] * 18 + [_i64] * 6 + [_int, _int, _int, _vp]
    lib.mq_moe_layer.restype = _int
    lib.mq_moe_layer.argtypes = [_vp] * 14 + [_i64] * 6 + [_int, _int, _int, _vp]
    lib.mq_swiglu.restype = _int
    lib.mq_swiglu.argtypes = [_vp, _vp, _vp, _i64, _int, _vp]
    lib.mq_moe_combine_shared.restype = _int
    lib.mq_moe_combine_shared.argtypes = [_vp, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64,
                                          _int, _vp]
    lib.mq_moe_route.restype = _int
    lib.mq_moe_route.argtypes = [_vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _int, _vp]
    lib.mq_gather_glu.restype = _int
    lib.mq_gather_glu.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64,
                                  _i64, _i64, _i64, _i64, _int, _int, _int, _vp, ctypes.c_size_t,
                                  _vp]
    lib.mq_gather_qmm_combine.restype = _int
    lib.mq_gather_qmm_combine.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64,
                                          _i64, _i64, _i64, _i64, _int, _int, _int, _vp]
    lib.mq_moe_combine.restype = _int
    lib.mq_moe_combine.argtypes = [_vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _int, _vp]


def lib() -> ctypes.CDLL:
    """Load the HIP library once; raise :class:`LibraryMissing` if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise LibraryMissing(
                    f"{LIB_PATH} is not built; run `python -m mlxturbo_amd.build` "
                    "(hipcc for gfx950).  mlxturbo_amd has no CPU fallback.")
            handle = ctypes.CDLL(LIB_PATH)
            _bind(handle)
            _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    """Map an ABI status to the exception MLX would raise."""
    if rc == MQ_OK:
        return
    msg = lib().mq_last_error().decode(errors="replace")
    if rc == MQ_EINVAL:
        raise ValueError(f"[{what}] {msg}")
    if rc == MQ_EUNSUPPORTED:
        raise NotImplementedError(f"[{what}] {msg}")
    raise RuntimeError(f"[{what}] HIP error {rc}: {msg}")


def launch_count() -> int:
    return int(lib().mq_launch_count())
