"""ctypes wrapper over oracle/liboracle.so -- TEST INFRASTRUCTURE ONLY.

The oracle restates the reference's INT8 linear kernels on the CPU
(kernel/w8a32_kernel.c, kernel/w8a8_kernel.c, kernel/w8a16_kernel.c).  Only
tests/, the smoke check and bench.py's CPU-baseline leg use it, and only as
the checker or as the timed CPU baseline.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIBS: dict[str, ctypes.CDLL] = {}

_i8p = ctypes.POINTER(ctypes.c_int8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_i32p = ctypes.POINTER(ctypes.c_int32)
_f32p = ctypes.POINTER(ctypes.c_float)


def build(native: bool = False) -> Path:
    """Compile the oracle with its Makefile; returns the library path."""
    target = "native" if native else "all"
    subprocess.run(["make", "-s", "-C", str(_HERE), target], check=True)
    return _HERE / ("liboracle_native.so" if native else "liboracle.so")


def load(native: bool = False) -> ctypes.CDLL:
    key = "native" if native else "portable"
    if key in _LIBS:
        return _LIBS[key]
    path = _HERE / ("liboracle_native.so" if native else "liboracle.so")
    if not path.exists():
        build(native)
    lib = ctypes.CDLL(str(path))
    lib.orc_quantize_rows.argtypes = [_f32p, _i8p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    lib.orc_int_acc.argtypes = [_i8p, _i8p, _i32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    lib.orc_w8a32_linear.argtypes = [_f32p, _i8p, _f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int, ctypes.c_int, _i8p, _f32p, _i32p]
    lib.orc_w8a8_linear.argtypes = [_i8p, _f32p, _i8p, _f32p, _f32p, _f32p, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_int, ctypes.c_int]
    lib.orc_w8a16_linear.argtypes = [_u16p, _i8p, _f32p, _f32p, _f32p, ctypes.c_int,
                                     ctypes.c_int, ctypes.c_int, ctypes.c_int]
    lib.orc_w8a32_gemv_timed.argtypes = [_f32p, _i8p, _f32p, _f32p, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_int]
    for f in ("orc_quantize_rows", "orc_int_acc", "orc_w8a32_linear", "orc_w8a8_linear",
              "orc_w8a16_linear", "orc_w8a32_gemv_timed"):
        getattr(lib, f).restype = None
    _LIBS[key] = lib
    return lib


def _p(a: np.ndarray | None, ct):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.POINTER(ct))


def _threads(threads: int | None) -> int:
    return threads if threads else (os.cpu_count() or 1)


def quantize_rows(src: np.ndarray, clamp_main: bool = True):
    """Per-row quantizer; returns (int8 codes, fp32 scales)."""
    src = np.ascontiguousarray(src, dtype=np.float32)
    if src.ndim == 1:
        src = src[None, :]
    rows, cols = src.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty(rows, np.float32)
    load().orc_quantize_rows(_p(src, ctypes.c_float), _p(q, ctypes.c_int8), _p(s, ctypes.c_float),
                             rows, cols, 1 if clamp_main else 0)
    return q, s


def int_acc(x_q: np.ndarray, w: np.ndarray, threads: int | None = None) -> np.ndarray:
    x_q = np.ascontiguousarray(np.atleast_2d(x_q), dtype=np.int8)
    w = np.ascontiguousarray(w, dtype=np.int8)
    b, k = x_q.shape
    n = w.shape[0]
    acc = np.empty((b, n), np.int32)
    load().orc_int_acc(_p(x_q, ctypes.c_int8), _p(w, ctypes.c_int8), _p(acc, ctypes.c_int32),
                       b, n, k, _threads(threads))
    return acc


def w8a32_linear(x: np.ndarray, w: np.ndarray, scales: np.ndarray, bias=None,
                 threads: int | None = None, detail: bool = False):
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.int8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    b, k = x.shape
    n = w.shape[0]
    y = np.empty((b, n), np.float32)
    codes = np.empty(k, np.int8) if (detail and b == 1) else None
    xs = np.empty(1, np.float32) if (detail and b == 1) else None
    acc = np.empty(n, np.int32) if (detail and b == 1) else None
    load().orc_w8a32_linear(_p(x, ctypes.c_float), _p(w, ctypes.c_int8), _p(scales, ctypes.c_float),
                            _p(bias, ctypes.c_float), _p(y, ctypes.c_float), b, n, k,
                            _threads(threads), _p(codes, ctypes.c_int8), _p(xs, ctypes.c_float),
                            _p(acc, ctypes.c_int32))
    if detail and b == 1:
        return y, codes, xs[0], acc
    return y


def w8a8_linear(x_q: np.ndarray, x_scales: np.ndarray, w: np.ndarray, w_scales: np.ndarray,
                bias=None, threads: int | None = None) -> np.ndarray:
    x_q = np.ascontiguousarray(np.atleast_2d(x_q), dtype=np.int8)
    x_scales = np.ascontiguousarray(np.atleast_1d(x_scales), dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.int8)
    w_scales = np.ascontiguousarray(w_scales, dtype=np.float32)
    bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    b, k = x_q.shape
    n = w.shape[0]
    y = np.empty((b, n), np.float32)
    load().orc_w8a8_linear(_p(x_q, ctypes.c_int8), _p(x_scales, ctypes.c_float), _p(w, ctypes.c_int8),
                           _p(w_scales, ctypes.c_float), _p(bias, ctypes.c_float),
                           _p(y, ctypes.c_float), b, n, k, _threads(threads))
    return y


def w8a16_linear(x_bf16: np.ndarray, w: np.ndarray, w_scales: np.ndarray, bias=None,
                 threads: int | None = None) -> np.ndarray:
    """x_bf16: uint16 raw bf16 bits [batch, K]."""
    x_bf16 = np.ascontiguousarray(np.atleast_2d(x_bf16), dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.int8)
    w_scales = np.ascontiguousarray(w_scales, dtype=np.float32)
    bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    b, k = x_bf16.shape
    n = w.shape[0]
    y = np.empty((b, n), np.float32)
    load().orc_w8a16_linear(_p(x_bf16, ctypes.c_uint16), _p(w, ctypes.c_int8),
                            _p(w_scales, ctypes.c_float), _p(bias, ctypes.c_float),
                            _p(y, ctypes.c_float), b, n, k, _threads(threads))
    return y


def w8a32_gemv_timed(x: np.ndarray, w: np.ndarray, scales: np.ndarray, y: np.ndarray,
                     threads: int, native: bool = False) -> None:
    """The CPU-baseline GEMV (same formula as w8a32_linear batch==1)."""
    n, k = w.shape
    load(native).orc_w8a32_gemv_timed(_p(x, ctypes.c_float), _p(w, ctypes.c_int8),
                                      _p(scales, ctypes.c_float), _p(y, ctypes.c_float),
                                      n, k, threads)
