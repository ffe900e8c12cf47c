"""ctypes bindings of libtyphoon_linear.so (include/typhoon_linear.h).

Part 1 functions keep the reference's signatures and host-pointer semantics
(kernel/w8a32_kernel.c:63-68, :355-363; kernel/w8a8_kernel.c:102-114,
:270-272; kernel/w8a16_kernel.c:44, :218-219).  The numpy wrappers below check
tl_last_error() after each call and raise RuntimeError, since the C functions
return void as in the reference.  There is no fallback: if the library is
missing or the GPU call fails, the wrapper raises.
"""
from __future__ import annotations

import ctypes
import os
from typing import List, Optional

import numpy as np

from . import LIB_PATH

_i8p = ctypes.POINTER(ctypes.c_int8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_i32p = ctypes.POINTER(ctypes.c_int32)
_f32p = ctypes.POINTER(ctypes.c_float)
_vp = ctypes.c_void_p
_int = ctypes.c_int

TL_F32, TL_BF16, TL_F16 = 0, 1, 2

# name -> (restype, argtypes); Part 1 first, then Part 2
SIGNATURES = {
    "w8a32_quantize": (None, [_f32p, _i8p, _f32p, _int, _int]),
    "w8a32_linear": (None, [_f32p, _i8p, _f32p, _f32p, _f32p, _f32p, _int, _int, _int]),
    "w8a8_quantize_weights": (None, [_f32p, _i8p, _f32p, _int, _int]),
    "w8a8_quantize_activations": (None, [_f32p, _i8p, _f32p, _int, _int]),
    "w8a8_linear": (None, [_i8p, _f32p, _i8p, _f32p, _f32p, _f32p, _int, _int, _int]),
    "w8a16_quantize_weights": (None, [_f32p, _i8p, _f32p, _int, _int]),
    "w8a16_linear": (None, [_u16p, _i8p, _f32p, _f32p, _f32p, _int, _int, _int]),
    "tl_last_error": (ctypes.c_char_p, []),
    "tl_clear_error": (None, []),
    "tl_version": (ctypes.c_char_p, []),
    "tl_device_count": (_int, []),
    "tl_gemv_set_plan": (_int, [_int, _int]),
    "tl_gemm_i8_set_cfg": (_int, [_int]),
    "tl_gemm_i8_set_split": (_int, [_int]),
    "tl_gemm_b16_set_plan": (_int, [_int, _int]),
    "tl_rows_set_split": (_int, [_int]),
    "tl_rows_set_groups": (_int, [_int]),
    "tl_w8a16_set_gemv": (_int, [_int]),
    "tl_w8a32_set_gemv2": (_int, [_int]),
    "tl_attn_set_chunk": (_int, [_int]),
    "tl_prefill_set_fused_quant": (_int, [_int]),
    "tl_stream_read_dev": (_int, [_vp, ctypes.c_size_t, _int, _int, _vp, _vp]),
    "tl_gemv_fused_dev": (_int, [_vp, _vp, _vp, _vp, _int, _int, _vp, _vp]),
    # decoder loop (Part 3), reference argtypes (decoder.py:86-143)
    "decoder_model_alloc": (_vp, []),
    "decoder_model_free": (None, [_vp]),
    "decoder_cache_alloc": (_vp, [_int]),
    "decoder_cache_free": (None, [_vp]),
    "decoder_cache_clear": (None, [_vp]),
    "decoder_cache_set_rope_offset": (None, [_vp, _int]),
    "decoder_scratch_alloc_fn": (_vp, [_int]),
    "decoder_scratch_free_fn": (None, [_vp]),
    "decoder_set_layer_weights": (None, [_vp, _int] + [_i8p, _f32p] * 7 + [_f32p] * 4),
    "decoder_set_layer_weights_v32": (None, [_vp, _int] + [_i8p, _f32p] * 7 + [_f32p] * 4 + [_i8p, _f32p] * 2),
    "decoder_precompute_rope": (None, [_f32p, _f32p, _int, _int, ctypes.POINTER(ctypes.c_int), _f32p]),
    "decoder_decode_step": (None, [_vp, _vp, _f32p, _vp, _f32p, _f32p]),
    "decoder_prefill_step": (None, [_vp, _vp, _f32p, _vp, _f32p, _f32p, _int]),
    "decoder_chunked_prefill_step": (None, [_vp, _vp, _f32p, _vp, _f32p, _f32p, _int, _int]),
    "decoder_hybrid_chunked_prefill_step": (None, [_vp, _vp, _f32p, _vp, _f32p, _f32p, _int, _int]),
    "decoder_prefill_step_3d": (None, [_vp, _vp, _f32p, _vp, _f32p, _f32p, _int]),
    "decoder_build_rope_3d": (None, [_f32p, _f32p, ctypes.POINTER(ctypes.c_int), _int, _int,
                                     ctypes.POINTER(ctypes.c_int), _f32p]),
    "tl_decoder_num_layers": (_int, [_vp]),
    "tl_decoder_cache_len": (_int, [_vp]),
    "tl_decoder_set_prefill_w8a8": (_int, [_vp, _int]),
    "tl_decoder_read_cache": (_int, [_vp, _int, _f32p, _f32p]),
    "tl_decoder_generate": (_int, [_vp, _vp, _vp, _vp, _f32p, _vp, _int, _int,
                                   ctypes.POINTER(ctypes.c_int32), _f32p, _f32p]),
    "tl_weights_save": (_int, [_vp, ctypes.c_char_p, ctypes.c_char_p, _int]),
    "tl_weights_load": (_vp, [ctypes.c_char_p, ctypes.c_char_p]),
    "tl_weights_cache_list": (_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_size_t]),
    "tl_weights_export": (_int, [_vp, _vp, _vp, _int]),
    "tl_registry_adopt": (_int, [_i8p, _f32p, _vp]),
    "tl_register_weights": (_int, [_i8p, _f32p, _int, _int]),
    "tl_evict_weights": (_int, [_i8p]),
    "tl_registry_clear": (None, []),
    "tl_registry_bytes": (ctypes.c_size_t, []),
    "tl_registry_entries": (_int, []),
    "tl_weights_create": (_vp, [_vp, _vp, _int, _int, _int]),
    "tl_weights_quantize_dev": (_vp, [_vp, _int, _int, _vp, _vp, _vp]),
    "tl_weights_destroy": (None, [_vp]),
    "tl_weights_rows": (_int, [_vp]),
    "tl_weights_cols": (_int, [_vp]),
    "tl_weights_bytes": (ctypes.c_size_t, [_vp]),
    "tl_w8a32_linear_dev": (_int, [_vp, _vp, _vp, _vp, _int, _vp]),
    "tl_quantize_rows_dev": (_int, [_vp, _vp, _vp, _int, _int, _int, _vp]),
    "tl_w8a8_linear_dev": (_int, [_vp, _vp, _vp, _vp, _vp, _int, _vp]),
    "tl_w8a8_linear_f32_dev": (_int, [_vp, _vp, _vp, _vp, _int, _vp]),
    "tl_w8a8_tiles_bytes": (ctypes.c_size_t, [_int, _int]),
    "tl_w8a8_quantize_tiles_dev": (_int, [_vp, _int, _int, _vp, _vp, _vp]),
    "tl_w8a8_linear_tiles_dev": (_int, [_vp, _vp, _vp, _vp, _vp, _int, _vp]),
    "tl_w8a16_linear_dev": (_int, [_vp, _int, _vp, _vp, _vp, _int, _int, _vp]),
    "tl_w8a32_gemv_acc_dev": (_int, [_vp, _vp, _vp, _vp, _vp]),
    "tl_w8a8_gemm_acc_dev": (_int, [_vp, _vp, _vp, _int, _vp]),
    "tl_lm_head_argmax_dev": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "tl_lm_head_argmax_noalloc_dev": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "tl_lm_head_argmax": (_int, [_f32p, _f32p, _i8p, _f32p, _int, _int, _f32p, ctypes.POINTER(ctypes.c_int32)]),
    "tl_rmsnorm_np_dev": (_int, [_vp, _vp, _vp, _int, _vp]),
    "tl_attn_decode_dev": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _int, _int, _int, _vp, _vp]),
    "tl_attn_prefill_dev": (_int, [_vp, _vp, _vp, _vp, _int, _int, _int, _int, _int, _vp]),
}

_LIB: Optional[ctypes.CDLL] = None


def load_library(path=None) -> ctypes.CDLL:
    """Load libtyphoon_linear.so and declare every exported signature."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = path or LIB_PATH
    # torch ships its own HIP/HSA runtime (same SONAME libamdhip64.so.7 as
    # /opt/rocm's).  Loading torch first makes this library bind to that one
    # runtime; loading it first would make a later `import torch` bring a
    # second runtime into the process, which then sees no GPU.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    if not p.exists():
        raise RuntimeError(f"{p} is missing: build it first (make -C {p.parent})")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _LIB = lib
    return lib


def check(lib: ctypes.CDLL, what: str) -> None:
    msg = lib.tl_last_error()
    if msg:
        raise RuntimeError(f"{what}: {msg.decode()}")


def _p(a: Optional[np.ndarray], ct):
    if a is None:
        return None
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("array must be C-contiguous")
    return a.ctypes.data_as(ctypes.POINTER(ct))


# ---------------------------------------------------------------------------
# numpy wrappers over Part 1 (host pointers)
# ---------------------------------------------------------------------------
def quantize(w: np.ndarray, which: str = "w8a32_quantize"):
    """Per-row quantization via one of the four reference quantizers."""
    lib = load_library()
    w = np.ascontiguousarray(np.atleast_2d(w), dtype=np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty(rows, np.float32)
    getattr(lib, which)(_p(w, ctypes.c_float), _p(q, ctypes.c_int8), _p(s, ctypes.c_float), rows, cols)
    check(lib, which)
    return q, s


def w8a32_linear(x: np.ndarray, w: np.ndarray, scales: np.ndarray, bias=None,
                 out: Optional[np.ndarray] = None) -> np.ndarray:
    lib = load_library()
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    batch, K = x.shape
    M = w.shape[0]
    y = out if out is not None else np.empty((batch, M), np.float32)
    lib.w8a32_linear(_p(x, ctypes.c_float), _p(w, ctypes.c_int8), _p(scales, ctypes.c_float),
                     _p(bias, ctypes.c_float), _p(y, ctypes.c_float), None, batch, M, K)
    check(lib, "w8a32_linear")
    return y


def w8a8_linear(x_q: np.ndarray, x_scales: np.ndarray, w: np.ndarray, w_scales: np.ndarray,
                bias=None) -> np.ndarray:
    lib = load_library()
    x_q = np.ascontiguousarray(np.atleast_2d(x_q), dtype=np.int8)
    x_scales = np.ascontiguousarray(np.atleast_1d(x_scales), dtype=np.float32)
    batch, K = x_q.shape
    M = w.shape[0]
    y = np.empty((batch, M), np.float32)
    lib.w8a8_linear(_p(x_q, ctypes.c_int8), _p(x_scales, ctypes.c_float), _p(w, ctypes.c_int8),
                    _p(w_scales, ctypes.c_float), _p(bias, ctypes.c_float), _p(y, ctypes.c_float),
                    batch, M, K)
    check(lib, "w8a8_linear")
    return y


def w8a16_linear(x_bf16: np.ndarray, w: np.ndarray, w_scales: np.ndarray, bias=None) -> np.ndarray:
    lib = load_library()
    x_bf16 = np.ascontiguousarray(np.atleast_2d(x_bf16), dtype=np.uint16)
    batch, K = x_bf16.shape
    M = w.shape[0]
    y = np.empty((batch, M), np.float32)
    lib.w8a16_linear(_p(x_bf16, ctypes.c_uint16), _p(w, ctypes.c_int8), _p(w_scales, ctypes.c_float),
                     _p(bias, ctypes.c_float), _p(y, ctypes.c_float), batch, M, K)
    check(lib, "w8a16_linear")
    return y


# ---------------------------------------------------------------------------
# Part 2 helpers over torch device tensors (torch is only the allocator here)
# ---------------------------------------------------------------------------
def _ptr(t) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(stream) -> Optional[int]:
    if stream is None:
        import torch
        stream = torch.cuda.current_stream()
    return stream.cuda_stream


class DeviceWeights:
    """Packed int8 tiles + fp32 scales resident in HBM (tl_weights)."""

    def __init__(self, handle: int, rows: int, cols: int):
        self.handle = handle
        self.rows = rows
        self.cols = cols

    @classmethod
    def from_codes(cls, w_int8, scales) -> "DeviceWeights":
        """w_int8/scales: torch device tensors or numpy host arrays."""
        lib = load_library()
        if isinstance(w_int8, np.ndarray):
            w_int8 = np.ascontiguousarray(w_int8, dtype=np.int8)
            scales = np.ascontiguousarray(scales, dtype=np.float32)
            rows, cols = w_int8.shape
            h = lib.tl_weights_create(w_int8.ctypes.data, scales.ctypes.data, rows, cols, 0)
        else:
            w_int8 = w_int8.contiguous()
            scales = scales.contiguous()
            rows, cols = w_int8.shape
            h = lib.tl_weights_create(w_int8.data_ptr(), scales.data_ptr(), rows, cols, 1)
        if not h:
            check(lib, "tl_weights_create")
            raise RuntimeError("tl_weights_create failed")
        return cls(h, rows, cols)

    @classmethod
    def quantize(cls, w_fp32, codes_out=None, scales_out=None, stream=None) -> "DeviceWeights":
        lib = load_library()
        rows, cols = w_fp32.shape
        h = lib.tl_weights_quantize_dev(w_fp32.data_ptr(), rows, cols, _ptr(codes_out), _ptr(scales_out),
                                        _stream(stream))
        if not h:
            check(lib, "tl_weights_quantize_dev")
            raise RuntimeError("tl_weights_quantize_dev failed")
        return cls(h, rows, cols)

    @classmethod
    def load(cls, path: str, name: str) -> "DeviceWeights":
        """Record `name` of a packed-weight cache file, copied into HBM."""
        lib = load_library()
        h = lib.tl_weights_load(os.fsencode(path), name.encode())
        if not h:
            check(lib, "tl_weights_load")
            raise RuntimeError("tl_weights_load failed")
        return cls(h, lib.tl_weights_rows(h), lib.tl_weights_cols(h))

    def save(self, path: str, name: str, append: bool = True) -> None:
        """Write this matrix as record `name` of a packed-weight cache file."""
        lib = load_library()
        _rc(lib, lib.tl_weights_save(self.handle, os.fsencode(path), name.encode(), int(append)),
            "tl_weights_save")

    def export(self):
        """(row-major int8 codes [rows, cols], fp32 scales [rows]) as numpy arrays."""
        lib = load_library()
        codes = np.empty((self.rows, self.cols), dtype=np.int8)
        scales = np.empty(self.rows, dtype=np.float32)
        _rc(lib, lib.tl_weights_export(self.handle, codes.ctypes.data, scales.ctypes.data, 0),
            "tl_weights_export")
        return codes, scales

    def adopt_into_registry(self, codes: np.ndarray, scales: np.ndarray) -> None:
        """Hand this device copy to the host-pointer registry for the host
        arrays (codes, scales) that hold its contents; this object no longer
        owns it afterwards."""
        lib = load_library()
        _rc(lib, lib.tl_registry_adopt(_p(codes, ctypes.c_int8), _p(scales, ctypes.c_float), self.handle),
            "tl_registry_adopt")
        self.handle = None

    def bytes(self) -> int:
        return load_library().tl_weights_bytes(self.handle)

    def close(self):
        if self.handle:
            load_library().tl_weights_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def cache_list(path: str) -> List[str]:
    """Record names of a packed-weight cache file, in file order."""
    lib = load_library()
    n = lib.tl_weights_cache_list(os.fsencode(path), None, 0)
    if n < 0:
        check(lib, "tl_weights_cache_list")
        raise RuntimeError("tl_weights_cache_list failed")
    buf = ctypes.create_string_buffer(4097 * (n + 1))   # names are < 4096 bytes each
    _rc(lib, 0 if lib.tl_weights_cache_list(os.fsencode(path), buf, len(buf)) >= 0 else -1,
        "tl_weights_cache_list")
    return buf.value.decode().split("\n")[:n]


def _rc(lib, rc, what):
    if rc != 0:
        check(lib, what)
        raise RuntimeError(f"{what} failed")


def w8a32_linear_dev(x, W: DeviceWeights, y, bias=None, stream=None):
    lib = load_library()
    _rc(lib, lib.tl_w8a32_linear_dev(x.data_ptr(), W.handle, _ptr(bias), y.data_ptr(), x.shape[0],
                                     _stream(stream)), "tl_w8a32_linear_dev")


def w8a8_linear_f32_dev(x, W: DeviceWeights, y, bias=None, stream=None):
    lib = load_library()
    _rc(lib, lib.tl_w8a8_linear_f32_dev(x.data_ptr(), W.handle, _ptr(bias), y.data_ptr(), x.shape[0],
                                        _stream(stream)), "tl_w8a8_linear_f32_dev")


def w8a8_quantize_tiles_dev(x, tiles, scales, stream=None):
    """Per-token int8 codes of fp32 x [M, K] into the activation tile layout
    (tiles: uint8 tensor of tl_w8a8_tiles_bytes(M, K) bytes; scales: fp32
    tensor of ceil(M / 16) * 16)."""
    lib = load_library()
    M, K = x.shape
    _rc(lib, lib.tl_w8a8_quantize_tiles_dev(x.data_ptr(), M, K, tiles.data_ptr(), scales.data_ptr(),
                                            _stream(stream)), "tl_w8a8_quantize_tiles_dev")


def w8a8_linear_tiles_dev(tiles, scales, W: DeviceWeights, y, bias=None, stream=None):
    """The W8A8 GEMM on tiled activation codes (w8a8_quantize_tiles_dev)."""
    lib = load_library()
    _rc(lib, lib.tl_w8a8_linear_tiles_dev(tiles.data_ptr(), scales.data_ptr(), W.handle, _ptr(bias),
                                          y.data_ptr(), y.shape[0], _stream(stream)), "tl_w8a8_linear_tiles_dev")


def w8a8_linear_dev(x_q, x_scales, W: DeviceWeights, y, bias=None, stream=None):
    lib = load_library()
    _rc(lib, lib.tl_w8a8_linear_dev(x_q.data_ptr(), x_scales.data_ptr(), W.handle, _ptr(bias),
                                    y.data_ptr(), x_q.shape[0], _stream(stream)), "tl_w8a8_linear_dev")


def w8a16_linear_dev(x, W: DeviceWeights, y, bias=None, stream=None):
    import torch
    lib = load_library()
    xt = TL_BF16 if x.dtype == torch.bfloat16 else TL_F16
    yt = {torch.float32: TL_F32, torch.bfloat16: TL_BF16, torch.float16: TL_F16}[y.dtype]
    _rc(lib, lib.tl_w8a16_linear_dev(x.data_ptr(), xt, W.handle, _ptr(bias), y.data_ptr(), yt,
                                     x.shape[0], _stream(stream)), "tl_w8a16_linear_dev")


def quantize_rows_dev(src, codes, scales, clamp127=True, stream=None):
    lib = load_library()
    rows, cols = src.shape
    _rc(lib, lib.tl_quantize_rows_dev(src.data_ptr(), codes.data_ptr(), scales.data_ptr(), rows, cols,
                                      1 if clamp127 else 0, _stream(stream)), "tl_quantize_rows_dev")


def gemv_acc_dev(x, W: DeviceWeights, acc, x_scale=None, stream=None):
    lib = load_library()
    _rc(lib, lib.tl_w8a32_gemv_acc_dev(x.data_ptr(), W.handle, acc.data_ptr(), _ptr(x_scale),
                                       _stream(stream)), "tl_w8a32_gemv_acc_dev")


def gemm_acc_dev(x_q, W: DeviceWeights, acc, stream=None):
    lib = load_library()
    _rc(lib, lib.tl_w8a8_gemm_acc_dev(x_q.data_ptr(), W.handle, acc.data_ptr(), x_q.shape[0],
                                      _stream(stream)), "tl_w8a8_gemm_acc_dev")


def gemv_fused_dev(x, W: DeviceWeights, y, epi=0, norm=0, norm_w=None, bias=None, stream=None):
    """The M=1 GEMV with the decoder's fusions (tl_gemv_fused_dev)."""
    lib = load_library()
    _rc(lib, lib.tl_gemv_fused_dev(x.data_ptr(), W.handle, _ptr(bias), y.data_ptr(), epi, norm, _ptr(norm_w),
                                   _stream(stream)), "tl_gemv_fused_dev")


def lm_head_argmax_dev(h, norm_w, W: DeviceWeights, token, logits=None, max_logit=None, stream=None):
    """Greedy token from the last hidden row h [K] (device tensors): final
    RMSNorm (numpy's float32 order), lm_head GEMV, argmax, into token (int32[1])."""
    lib = load_library()
    _rc(lib, lib.tl_lm_head_argmax_dev(h.data_ptr(), _ptr(norm_w), W.handle, _ptr(logits), token.data_ptr(),
                                       _ptr(max_logit), _stream(stream)), "tl_lm_head_argmax_dev")


def lm_head_argmax_noalloc_dev(h, norm_w, W: DeviceWeights, token, logits=None, max_logit=None, stream=None):
    """lm_head_argmax_dev with the library's fixed device work-space: no
    device allocation, lm_heads of up to 262144 rows and K up to 16384."""
    lib = load_library()
    _rc(lib, lib.tl_lm_head_argmax_noalloc_dev(h.data_ptr(), _ptr(norm_w), W.handle, _ptr(logits),
                                               token.data_ptr(), _ptr(max_logit), _stream(stream)),
        "tl_lm_head_argmax_noalloc_dev")


def lm_head_argmax(h: np.ndarray, norm_w: Optional[np.ndarray], w: np.ndarray, scales: np.ndarray,
                   logits: Optional[np.ndarray] = None) -> int:
    """Host-pointer variant: returns the greedy token id."""
    lib = load_library()
    h = np.ascontiguousarray(h, dtype=np.float32).reshape(-1)
    nw = None if norm_w is None else np.ascontiguousarray(norm_w, dtype=np.float32)
    tok = ctypes.c_int32(-1)
    rc = lib.tl_lm_head_argmax(_p(h, ctypes.c_float), _p(nw, ctypes.c_float), _p(w, ctypes.c_int8),
                               _p(scales, ctypes.c_float), w.shape[0], w.shape[1], _p(logits, ctypes.c_float),
                               ctypes.byref(tok))
    if rc != 0:
        check(lib, "tl_lm_head_argmax")
    return int(tok.value)


def rmsnorm_np_dev(h, norm_w, out, stream=None):
    lib = load_library()
    _rc(lib, lib.tl_rmsnorm_np_dev(h.data_ptr(), _ptr(norm_w), out.data_ptr(), h.numel(), _stream(stream)),
        "tl_rmsnorm_np_dev")
