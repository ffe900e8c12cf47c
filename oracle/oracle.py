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
    lib.orc_base_w8a32_gemm.argtypes = [_f32p, _i8p, _f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_int]
    lib.orc_base_w8a8_gemm.argtypes = [_i8p, _f32p, _i8p, _f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_int, ctypes.c_int]
    lib.orc_base_w8a16_linear.argtypes = [_u16p, _i8p, _f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int, ctypes.c_int]
    for f in ("orc_quantize_rows", "orc_int_acc", "orc_w8a32_linear", "orc_w8a8_linear",
              "orc_w8a16_linear", "orc_w8a32_gemv_timed", "orc_base_w8a32_gemm", "orc_base_w8a8_gemm",
              "orc_base_w8a16_linear"):
        getattr(lib, f).restype = None
    _f = ctypes.c_float
    _i = ctypes.c_int
    for f in ("orc_frecpe", "orc_frsqrte", "orc_fast_exp", "orc_silu_fast"):
        getattr(lib, f).argtypes = [_f]
        getattr(lib, f).restype = _f
    for f in ("orc_frecps", "orc_frsqrts"):
        getattr(lib, f).argtypes = [_f, _f]
        getattr(lib, f).restype = _f
    lib.orc_rmsnorm.argtypes = [_f32p, _f32p, _f32p, _i, _f]
    lib.orc_mrope_precompute.argtypes = [_f32p, _f32p, _i, _i, _f]
    lib.orc_mrope_apply.argtypes = [_f32p, _f32p, _f32p, _f32p, _i, _i, _i, _i]
    lib.orc_silu_mul.argtypes = [_f32p, _f32p, _i]
    lib.orc_attention_decode.argtypes = [_f32p, _f32p, _f32p, _f32p, _i, _i, _i, _i, _f]
    lib.orc_decode_layer.argtypes = [ctypes.POINTER(_i8p), ctypes.POINTER(_f32p), _f32p, _f32p, _f32p, _f32p,
                                     _f32p, _f32p, _i, _f32p, _f32p, _f32p, _i, _i, _i, _i, _i, _i, _i]
    lib.orc_mrope_build_3d.argtypes = [_f32p, _f32p, _i32p, _i, _i, _i32p, _f]
    lib.orc_attention_prefill.argtypes = [_f32p, _f32p, _f32p, _f32p, _i, _i, _i, _f]
    lib.orc_prefill_layer.argtypes = [ctypes.POINTER(_i8p), ctypes.POINTER(_f32p), _f32p, _f32p, _f32p, _f32p,
                                      _f32p, _f32p, _i, _f32p, _i, _f32p, _f32p, _f32p, _f32p, _i, _i, _i, _i,
                                      _i, _i, _i]
    for f in ("orc_rmsnorm", "orc_mrope_precompute", "orc_mrope_apply", "orc_silu_mul",
              "orc_attention_decode", "orc_decode_layer", "orc_mrope_build_3d", "orc_attention_prefill",
              "orc_prefill_layer"):
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


def base_w8a32_gemm(x, w, scales, threads: int, native: bool = False, bias=None) -> np.ndarray:
    """The CPU baseline's w8a32_linear at batch > 1 (64-row dequantized tiles, blocked SGEMM)."""
    x = np.ascontiguousarray(x, np.float32)
    bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
    m, k = x.shape
    n = w.shape[0]
    y = np.empty((m, n), np.float32)
    load(native).orc_base_w8a32_gemm(_p(x, ctypes.c_float), _p(w, ctypes.c_int8), _p(scales, ctypes.c_float),
                                     _p(bias, ctypes.c_float), _p(y, ctypes.c_float), m, n, k, threads)
    return y


def base_w8a8_gemm(x_q, x_scales, w, w_scales, threads: int, native: bool = False, bias=None) -> np.ndarray:
    """The CPU baseline's w8a8_linear at batch > 1 (X dequantized, 128-row tiles, blocked SGEMM)."""
    x_q = np.ascontiguousarray(x_q, np.int8)
    bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
    m, k = x_q.shape
    n = w.shape[0]
    y = np.empty((m, n), np.float32)
    load(native).orc_base_w8a8_gemm(_p(x_q, ctypes.c_int8), _p(x_scales, ctypes.c_float), _p(w, ctypes.c_int8),
                                    _p(w_scales, ctypes.c_float), _p(bias, ctypes.c_float),
                                    _p(y, ctypes.c_float), m, n, k, threads)
    return y


def base_w8a16_linear(x_bf16, w, w_scales, threads: int, native: bool = False, bias=None) -> np.ndarray:
    """The CPU baseline's w8a16_linear (batch 1: chunked GEMV; batch > 1: 128-row tiles, blocked SGEMM)."""
    x_bf16 = np.ascontiguousarray(x_bf16, np.uint16)
    bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
    m, k = x_bf16.shape
    n = w.shape[0]
    y = np.empty((m, n), np.float32)
    load(native).orc_base_w8a16_linear(_p(x_bf16, ctypes.c_uint16), _p(w, ctypes.c_int8),
                                       _p(w_scales, ctypes.c_float), _p(bias, ctypes.c_float),
                                       _p(y, ctypes.c_float), m, n, k, threads)
    return y


# ---------------------------------------------------------------------------
# decoder layer step (decoder_ref.c)
# ---------------------------------------------------------------------------
HEAD_DIM = 128
ROPE_THETA = 5000000.0          # MROPE_THETA_BASE, reference decoder.py:41


def frecpe(x: float) -> float:
    return load().orc_frecpe(x)


def frsqrte(x: float) -> float:
    return load().orc_frsqrte(x)


def frecps(a: float, b: float) -> float:
    return load().orc_frecps(a, b)


def frsqrts(a: float, b: float) -> float:
    return load().orc_frsqrts(a, b)


def fast_exp(x: float) -> float:
    return load().orc_fast_exp(x)


def silu_fast(g: float) -> float:
    return load().orc_silu_fast(g)


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """rmsnorm_f32 over the last axis (rows independent)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.empty_like(x)
    dim = x.shape[-1]
    xr, orow = x.reshape(-1, dim), out.reshape(-1, dim)
    for r in range(xr.shape[0]):
        load().orc_rmsnorm(_p(orow[r], ctypes.c_float), _p(xr[r], ctypes.c_float), _p(w, ctypes.c_float),
                           dim, eps)
    return out


def rope_tables(max_seq: int, head_dim: int = HEAD_DIM, theta: float = ROPE_THETA):
    half = head_dim // 2
    c = np.empty((max_seq, half), np.float32)
    s_ = np.empty((max_seq, half), np.float32)
    load().orc_mrope_precompute(_p(c, ctypes.c_float), _p(s_, ctypes.c_float), max_seq, head_dim, theta)
    return c, s_


def mrope_apply(q: np.ndarray, k: np.ndarray, cos_tab, sin_tab, pos: int):
    """Returns rotated copies of q [nq*128] and k [nk*128] at position pos."""
    q = np.array(q, dtype=np.float32, copy=True)
    k = np.array(k, dtype=np.float32, copy=True)
    load().orc_mrope_apply(_p(q, ctypes.c_float), _p(k, ctypes.c_float), _p(cos_tab, ctypes.c_float),
                           _p(sin_tab, ctypes.c_float), q.size // HEAD_DIM, k.size // HEAD_DIM, HEAD_DIM, pos)
    return q, k


def silu_mul(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    g = np.array(gate, dtype=np.float32, copy=True)
    u = np.ascontiguousarray(up, dtype=np.float32)
    load().orc_silu_mul(_p(g, ctypes.c_float), _p(u, ctypes.c_float), g.size)
    return g


def attention_decode(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, S: int,
                     scale: float = 0.08838834764831843) -> np.ndarray:
    """q [nq*128]; kc/vc [nkv, max_seq, 128]; attends to positions 0..S-1."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    kc = np.ascontiguousarray(kc, dtype=np.float32)
    vc = np.ascontiguousarray(vc, dtype=np.float32)
    nkv, max_seq, _ = kc.shape
    out = np.empty_like(q)
    load().orc_attention_decode(_p(q, ctypes.c_float), _p(kc, ctypes.c_float), _p(vc, ctypes.c_float),
                                _p(out, ctypes.c_float), q.size // HEAD_DIM, nkv, max_seq, S, scale)
    return out


LAYER_PROJ = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


def decode_layer(layer: dict, kc: np.ndarray, vc: np.ndarray, hidden: np.ndarray, cos_tab, sin_tab,
                 cache_len: int, rope_pos: int, threads: int | None = None) -> np.ndarray:
    """One DECODE_MODE layer.  layer: name -> (int8 codes, fp32 scales) for
    the seven projections, plus input_ln / post_attn_ln / q_norm / k_norm
    fp32 vectors.  kc/vc: this layer's cache [nkv, max_seq, 128], updated in
    place at position cache_len.  Returns the new hidden row."""
    h = np.array(hidden, dtype=np.float32, copy=True).reshape(-1)
    ws = [np.ascontiguousarray(layer[n][0], dtype=np.int8) for n in LAYER_PROJ]
    ss = [np.ascontiguousarray(layer[n][1], dtype=np.float32) for n in LAYER_PROJ]
    norms = [np.ascontiguousarray(layer[n], dtype=np.float32)
             for n in ("input_ln", "post_attn_ln", "q_norm", "k_norm")]
    assert kc.flags["C_CONTIGUOUS"] and vc.flags["C_CONTIGUOUS"] and kc.dtype == np.float32
    nkv, max_seq, _ = kc.shape
    warr = (_i8p * 7)(*[_p(w, ctypes.c_int8) for w in ws])
    sarr = (_f32p * 7)(*[_p(s, ctypes.c_float) for s in ss])
    load().orc_decode_layer(warr, sarr, *[_p(n, ctypes.c_float) for n in norms], _p(kc, ctypes.c_float),
                            _p(vc, ctypes.c_float), max_seq, _p(h, ctypes.c_float),
                            _p(cos_tab, ctypes.c_float), _p(sin_tab, ctypes.c_float), cache_len, rope_pos,
                            h.size, ws[4].shape[0], ws[0].shape[0] // HEAD_DIM, nkv, _threads(threads))
    return h


def rope_tables_3d(pos_ids: np.ndarray, head_dim: int = HEAD_DIM, sections=(24, 20, 20),
                   theta: float = ROPE_THETA):
    """Per-token tables [S, head_dim/2] from pos_ids [3, S] (mrope_build_cos_sin_3d)."""
    pos = np.ascontiguousarray(pos_ids, dtype=np.int32)
    S = pos.shape[1]
    c = np.empty((S, head_dim // 2), np.float32)
    s_ = np.empty((S, head_dim // 2), np.float32)
    sec = (ctypes.c_int32 * 3)(*sections)
    load().orc_mrope_build_3d(_p(c, ctypes.c_float), _p(s_, ctypes.c_float), _p(pos, ctypes.c_int32), S, head_dim,
                              sec, theta)
    return c, s_


def attention_prefill(q: np.ndarray, k: np.ndarray, v: np.ndarray, nq: int = 16, nkv: int = 8,
                      scale: float = 0.08838834764831843) -> np.ndarray:
    """q [S, nq*128], k/v [S, nkv*128] token-major; causal within the chunk."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.empty_like(q)
    load().orc_attention_prefill(_p(q, ctypes.c_float), _p(k, ctypes.c_float), _p(v, ctypes.c_float),
                                 _p(out, ctypes.c_float), q.shape[0], nq, nkv, scale)
    return out


def prefill_layer(layer: dict, kc: np.ndarray, vc: np.ndarray, hidden: np.ndarray, cos_tab=None, sin_tab=None,
                  token_cos=None, token_sin=None, cache_len: int = 0, threads: int | None = None,
                  w8a8: bool = False) -> np.ndarray:
    """One PREFILL_MODE (cos_tab/sin_tab rows cache_len + t) or PREFILL_3D_MODE
    (token_cos/token_sin rows t) layer over hidden [S, H]; kc/vc updated in
    place.  w8a8: the linears on per-token int8 activations."""
    h = np.array(hidden, dtype=np.float32, copy=True)
    S, H = h.shape
    ws = [np.ascontiguousarray(layer[n][0], dtype=np.int8) for n in LAYER_PROJ]
    ss = [np.ascontiguousarray(layer[n][1], dtype=np.float32) for n in LAYER_PROJ]
    norms = [np.ascontiguousarray(layer[n], dtype=np.float32)
             for n in ("input_ln", "post_attn_ln", "q_norm", "k_norm")]
    nkv, max_seq, _ = kc.shape
    warr = (_i8p * 7)(*[_p(w, ctypes.c_int8) for w in ws])
    sarr = (_f32p * 7)(*[_p(s, ctypes.c_float) for s in ss])
    f = lambda a: None if a is None else _p(np.ascontiguousarray(a, dtype=np.float32), ctypes.c_float)
    load().orc_prefill_layer(warr, sarr, *[_p(n, ctypes.c_float) for n in norms], _p(kc, ctypes.c_float),
                             _p(vc, ctypes.c_float), max_seq, _p(h, ctypes.c_float), S, f(cos_tab), f(sin_tab),
                             f(token_cos), f(token_sin), cache_len, H, ws[4].shape[0], ws[0].shape[0] // HEAD_DIM,
                             nkv, _threads(threads), 1 if w8a8 else 0)
    return h
