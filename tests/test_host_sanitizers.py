"""The C host layer (csrc/api.c, csrc/decoder_host.c) built with
-fsanitize=address,undefined and driven through its argument checks and
error paths by tests/sanitize/host_errors.c, on the CPU: every entry point
reached without usable arguments (or without a device) must fail cleanly with
a message naming it, the packed-weight cache reader must list a valid file and
reject damaged ones, four threads must do the same concurrently, and the run
must end with no memory error, leak or undefined behaviour reported."""
import os
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

import wcache_format as fmt

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "typhoon-ocr-server_amd"
KERNEL_OBJS = ["quant", "gemv", "gemm", "gemm_i8", "gemm_b16", "gemm_small", "rows", "stream", "lmhead",
               "decoder", "prefill"]


def _w(rng, rows, cols):
    return rng.integers(-127, 128, (rows, cols), dtype=np.int8), rng.uniform(0.002, 0.02, rows).astype(np.float32)


def test_host_layer_error_paths_under_sanitizers(tmp_path):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    objs = [PKG / "_build" / f"{o}.o" for o in KERNEL_OBJS]
    if not all(o.exists() for o in objs):
        pytest.skip("kernel objects not built (run __graft_entry__.build() first)")
    exe = tmp_path / "host_errors"
    cmd = ["gcc", "-std=c11", "-g", "-O1", "-fsanitize=address,undefined", "-fno-omit-frame-pointer", "-pthread",
           "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", str(PKG / "csrc" / "api.c"),
           str(PKG / "csrc" / "decoder_host.c"), str(ROOT / "tests" / "sanitize" / "host_errors.c"),
           *map(str, objs), "-L/opt/rocm/lib", "-Wl,-rpath,/opt/rocm/lib", "-lamdhip64", "-lstdc++", "-lm",
           "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=300)

    rng = np.random.default_rng(5)
    good = tmp_path / "good.tlw"
    names = ["layers.0.o_proj", "lm_head"]
    good.write_bytes(b"".join(fmt.record(n, *_w(rng, 20 + 16 * i, 70 + 64 * i)) for i, n in enumerate(names)))
    damaged = []
    for damage in ("magic", "version", "shape", "sizes", "truncate"):
        rec = bytearray(fmt.record("m", *_w(rng, 33, 100)))
        if damage == "magic":
            rec[0:8] = b"NOTACACH"
        elif damage == "version":
            rec[8] = 9
        elif damage == "shape":
            rec[24:28] = (5).to_bytes(4, "little")
        elif damage == "sizes":
            rec[32] ^= 0x10
        else:
            rec = rec[:40]
        f = tmp_path / f"{damage}.tlw"
        f.write_bytes(bytes(rec))
        damaged.append(str(f))

    env = dict(os.environ)
    env["ASAN_OPTIONS"] = "detect_leaks=1:halt_on_error=1"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    r = subprocess.run([str(exe), str(good), "\n".join(names) + "\n", *damaged], env=env, capture_output=True,
                       text=True, timeout=300)
    assert "AddressSanitizer" not in r.stderr and "LeakSanitizer" not in r.stderr, r.stderr[-4000:]
    assert "runtime error" not in r.stderr, r.stderr[-4000:]
    assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-4000:])
    assert "0 failures" in r.stdout
