"""MI355X (gfx950) INT8 weight-quantized linear layers for typhoon-ocr-server.

The product is the C-ABI library libtyphoon_linear.so (include/typhoon_linear.h)
built from csrc/ by the Makefile next to this file.  The Python modules here
mirror the reference's Python side of that path:
  linear.py   ctypes bindings of the whole C ABI (+ numpy/torch helpers)
  decoder.py  load_decoder_lib() / Decoder linear-path mirror of the
              reference's decoder.py (weight quantization and packing at load,
              lm_head logits, greedy sampling)

The directory name is not a Python identifier; load it with
importlib (see __graft_entry__.py) under the name typhoon_ocr_server_amd.
"""
from pathlib import Path
import subprocess

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libtyphoon_linear.so"
HEADER = PKG_DIR.parent / "include" / "typhoon_linear.h"


def build(jobs: int = 8) -> Path:
    """Compile every HIP source for gfx950 and link libtyphoon_linear.so."""
    subprocess.run(["make", "-s", "-C", str(PKG_DIR), f"-j{jobs}"], check=True)
    if not LIB_PATH.exists():
        raise RuntimeError(f"build did not produce {LIB_PATH}")
    return LIB_PATH
