"""CPU checks of the drop-in boundary: the C-ABI library loads, exports every
function include/typhoon_linear.h declares, and the Python mirror binds the
reference's signatures.  No compute calls (no GPU here)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "typhoon_linear.h"

REFERENCE_ENTRY_POINTS = [
    "w8a32_quantize", "w8a32_linear", "w8a8_quantize_weights", "w8a8_quantize_activations",
    "w8a8_linear", "w8a16_quantize_weights", "w8a16_linear",
]


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b([A-Za-z_][A-Za-z0-9_]*)\s*\([^;{]*\)\s*;", text)
    return sorted(set(n for n in names if n not in ("if", "while", "sizeof")))


def test_header_declares_reference_entry_points():
    decl = declared_functions()
    for name in REFERENCE_ENTRY_POINTS:
        assert name in decl, name
    assert len(decl) >= 20


def test_library_exports_every_declared_symbol(pkg):
    lib = ctypes.CDLL(str(pkg.LIB_PATH))
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_bindings_cover_header(lin):
    assert set(lin.SIGNATURES) == set(declared_functions())
    lib = lin.load_library()
    assert lib.tl_version().decode().startswith("typhoon_linear")
    assert lib.tl_last_error() is None


def test_reference_argtypes(pkg):
    import importlib
    dec = importlib.import_module("typhoon_ocr_server_amd.decoder")
    lib = dec.load_decoder_lib()
    i8p, f32p = ctypes.POINTER(ctypes.c_int8), ctypes.POINTER(ctypes.c_float)
    # reference decoder.py:146-157
    assert lib.w8a32_quantize.argtypes == [f32p, i8p, f32p, ctypes.c_int, ctypes.c_int]
    assert lib.w8a32_linear.argtypes == [f32p, i8p, f32p, f32p, f32p, f32p,
                                         ctypes.c_int, ctypes.c_int, ctypes.c_int]


def test_missing_library_fails_loudly(lin, tmp_path):
    with pytest.raises(RuntimeError):
        lin.load_library(tmp_path / "libtyphoon_linear.so")


def test_bad_arguments_report_errors_without_gpu(lin):
    # argument validation happens before any device work and is reported
    # through tl_last_error (the reference functions return void)
    import numpy as np
    lib = lin.load_library()
    x = np.zeros((1, 16), np.float32)
    w = np.zeros((16, 16), np.int8)
    s = np.ones(16, np.float32)
    y = np.zeros((1, 16), np.float32)
    lib.w8a32_linear(lin._p(x, ctypes.c_float), lin._p(w, ctypes.c_int8), lin._p(s, ctypes.c_float),
                     None, lin._p(y, ctypes.c_float), None, 0, 16, 16)
    msg = lib.tl_last_error()
    assert msg is not None and b"batch" in msg
