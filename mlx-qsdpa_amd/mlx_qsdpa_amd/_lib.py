"""ctypes binding of the C ABI in include/qsdpa.h (libqsdpa_hip.so).

The library is built in-tree by ``mlx-qsdpa_amd/build_lib.py``.  Loading
fails loudly: there is no CPU or pure-PyTorch stand-in for the kernels.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libqsdpa_hip.so"

QSDPA_OK = 0
QSDPA_ERR_INVALID = -1
QSDPA_ERR_UNSUPPORTED = -2
QSDPA_ERR_WORKSPACE = -3
QSDPA_ERR_LAUNCH = -4

QSDPA_F16 = 0
QSDPA_BF16 = 1
QSDPA_F32 = 2
QSDPA_BOOL = 3

ABI_VERSION = 6
NOALLOC_SCRATCH_BYTES = 16 << 20

# Every symbol include/qsdpa.h declares.
EXPORTED_SYMBOLS = (
    "qsdpa_decode_workspace_size",
    "qsdpa_decode",
    "qsdpa_decode_noalloc",
    "qsdpa_quantize",
    "qsdpa_quantize_batch",
    "qsdpa_dequantize",
    "qsdpa_requant_window",
    "qsdpa_move_rows",
    "qsdpa_last_error",
    "qsdpa_abi_version",
)


class View(ctypes.Structure):
    _fields_ = [
        ("ptr", ctypes.c_void_p),
        ("stride_b", ctypes.c_int64),
        ("stride_h", ctypes.c_int64),
        ("stride_n", ctypes.c_int64),
    ]


class DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("B", ctypes.c_int32), ("H_q", ctypes.c_int32), ("H_kv", ctypes.c_int32),
        ("N", ctypes.c_int32), ("D", ctypes.c_int32),
        ("bits", ctypes.c_int32), ("group_size", ctypes.c_int32), ("dtype", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("q", View), ("k_packed", View), ("v_packed", View),
        ("k_scales", View), ("v_scales", View), ("k_biases", View), ("v_biases", View),
        ("out", View),
        ("mask", View), ("mask_dtype", ctypes.c_int32),
        ("kv_start", ctypes.c_void_p),
        ("num_splits", ctypes.c_int32),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("prof_begin", ctypes.c_void_p), ("prof_end", ctypes.c_void_p),
        ("q_len", ctypes.c_int32), ("causal", ctypes.c_int32), ("mask_stride_q", ctypes.c_int64),
        ("k_new", View), ("v_new", View),
    ]


class QuantizeArgs(ctypes.Structure):
    _fields_ = [
        ("B", ctypes.c_int32), ("H", ctypes.c_int32), ("S", ctypes.c_int32), ("D", ctypes.c_int32),
        ("bits", ctypes.c_int32), ("group_size", ctypes.c_int32), ("dtype", ctypes.c_int32),
        ("t0", ctypes.c_int32),
        ("src", View), ("dst_packed", View), ("dst_scales", View), ("dst_biases", View),
    ]


class DequantizeArgs(ctypes.Structure):
    _fields_ = [
        ("B", ctypes.c_int32), ("H", ctypes.c_int32), ("N", ctypes.c_int32), ("D", ctypes.c_int32),
        ("bits", ctypes.c_int32), ("group_size", ctypes.c_int32), ("dtype", ctypes.c_int32),
        ("keep", ctypes.c_int32), ("rot", ctypes.c_int32),
        ("src_packed", View), ("src_scales", View), ("src_biases", View), ("dst", View),
    ]


class RequantArgs(ctypes.Structure):
    _fields_ = [
        ("B", ctypes.c_int32), ("H", ctypes.c_int32), ("D", ctypes.c_int32),
        ("bits", ctypes.c_int32), ("group_size", ctypes.c_int32), ("dtype", ctypes.c_int32),
        ("n_old", ctypes.c_int32), ("keep", ctypes.c_int32), ("rot", ctypes.c_int32),
        ("S", ctypes.c_int32), ("max_size", ctypes.c_int32),
        ("old_packed", View), ("old_scales", View), ("old_biases", View), ("src", View),
        ("dst_packed", View), ("dst_scales", View), ("dst_biases", View),
    ]


class RowMove(ctypes.Structure):
    _fields_ = [
        ("src", ctypes.c_void_p), ("dst", ctypes.c_void_p),
        ("src_head_stride", ctypes.c_int64), ("src_token_stride", ctypes.c_int64),
        ("dst_head_stride", ctypes.c_int64), ("dst_token_stride", ctypes.c_int64),
        ("heads", ctypes.c_int32), ("tokens", ctypes.c_int32),
        ("row_bytes", ctypes.c_int32), ("copy_begin", ctypes.c_int32), ("copy_end", ctypes.c_int32),
    ]


class QsdpaError(RuntimeError):
    """Raised when a C-ABI call returns a negative status."""

    def __init__(self, code: int, message: str):
        super().__init__(f"qsdpa error {code}: {message}")
        self.code = code


_lib = None


def load(path: os.PathLike | str | None = None) -> ctypes.CDLL:
    """Load (once) and return the HIP library; raise if it is missing."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise ImportError(
            f"{p} is missing: build it with `python mlx-qsdpa_amd/build_lib.py` "
            "(the quantized SDPA path has no non-HIP fallback)")
    lib = ctypes.CDLL(str(p))
    lib.qsdpa_decode_workspace_size.argtypes = [ctypes.POINTER(DecodeArgs),
                                                ctypes.POINTER(ctypes.c_int32)]
    lib.qsdpa_decode_workspace_size.restype = ctypes.c_int64
    lib.qsdpa_decode.argtypes = [ctypes.POINTER(DecodeArgs), ctypes.c_void_p]
    lib.qsdpa_decode.restype = ctypes.c_int
    lib.qsdpa_decode_noalloc.argtypes = [ctypes.POINTER(DecodeArgs), ctypes.c_void_p]
    lib.qsdpa_decode_noalloc.restype = ctypes.c_int
    lib.qsdpa_quantize.argtypes = [ctypes.POINTER(QuantizeArgs), ctypes.c_void_p]
    lib.qsdpa_quantize.restype = ctypes.c_int
    lib.qsdpa_quantize_batch.argtypes = [ctypes.POINTER(QuantizeArgs), ctypes.c_int32, ctypes.c_void_p]
    lib.qsdpa_quantize_batch.restype = ctypes.c_int
    lib.qsdpa_dequantize.argtypes = [ctypes.POINTER(DequantizeArgs), ctypes.c_void_p]
    lib.qsdpa_dequantize.restype = ctypes.c_int
    lib.qsdpa_requant_window.argtypes = [ctypes.POINTER(RequantArgs), ctypes.c_int32, ctypes.c_void_p]
    lib.qsdpa_requant_window.restype = ctypes.c_int
    lib.qsdpa_move_rows.argtypes = [ctypes.POINTER(RowMove), ctypes.c_int32, ctypes.c_void_p]
    lib.qsdpa_move_rows.restype = ctypes.c_int
    lib.qsdpa_last_error.argtypes = []
    lib.qsdpa_last_error.restype = ctypes.c_char_p
    lib.qsdpa_abi_version.argtypes = []
    lib.qsdpa_abi_version.restype = ctypes.c_int
    ver = lib.qsdpa_abi_version()
    if ver != ABI_VERSION:
        raise ImportError(f"{p}: ABI version {ver}, expected {ABI_VERSION}")
    if path is None:
        _lib = lib
    return lib


def check(code: int) -> int:
    """Raise QsdpaError for a negative status; return it otherwise."""
    if code < 0:
        msg = load().qsdpa_last_error().decode(errors="replace")
        raise QsdpaError(int(code), msg)
    return code
