"""Packed-weight cache file: CPU checks of the reader (record listing and the
rejections that need no device) on files built by tests/wcache_format.py.
The GPU round trips are in tests/test_gpu_wcache.py."""
import numpy as np
import pytest

import wcache_format as fmt


def _w(rng, rows, cols):
    return rng.integers(-127, 128, (rows, cols), dtype=np.int8), rng.uniform(0.002, 0.02, rows).astype(np.float32)


def test_pack_tiles_layout():
    """The tile layout against its definition, element by element."""
    rng = np.random.default_rng(0)
    w, _ = _w(rng, 37, 130)
    t = np.frombuffer(fmt.pack_tiles(w), np.int8)
    NG, KB = 3, 3
    assert t.size == NG * KB * 1024
    for g in range(NG):
        for kb in range(KB):
            base = (kb * NG + g) * 1024
            for lane in range(64):
                for b in range(16):
                    r, k = 16 * g + (lane & 15), 64 * kb + 16 * (lane >> 4) + b
                    want = w[r, k] if r < 37 and k < 130 else 0
                    assert t[base + 16 * lane + b] == want


def test_checksum_detects_single_bit_flips():
    rng = np.random.default_rng(1)
    p = bytearray(rng.integers(0, 256, 4096, dtype=np.uint8).tobytes())
    h0 = fmt.checksum(bytes(p))
    for pos in (0, 7, 8, 31, 32, 1000, 4095):
        q = bytearray(p)
        q[pos] ^= 1
        assert fmt.checksum(bytes(q)) != h0


def test_list_records(lin, tmp_path):
    rng = np.random.default_rng(2)
    f = tmp_path / "w.tlw"
    names = ["layers.0.q_proj", "layers.0.k_proj", "lm_head"]
    f.write_bytes(b"".join(fmt.record(n, *_w(rng, 20 + 7 * i, 70 + 64 * i)) for i, n in enumerate(names)))
    assert lin.cache_list(str(f)) == names


@pytest.mark.parametrize("damage,msg", [
    ("magic", "bad magic"), ("version", "version"), ("shape", "inconsistent record shape"),
    ("sizes", "inconsistent record sizes"), ("truncate", "truncated"),
])
def test_reader_rejects_damaged_headers(lin, tmp_path, damage, msg):
    rng = np.random.default_rng(3)
    rec = bytearray(fmt.record("m", *_w(rng, 33, 100)))
    if damage == "magic":
        rec[0:8] = b"NOTACACH"
    elif damage == "version":
        rec[8] = 9
    elif damage == "shape":
        rec[24:28] = (5).to_bytes(4, "little")        # NG
    elif damage == "sizes":
        rec[32] ^= 0x10                                # tile_bytes
    else:
        rec = rec[:40]
    f = tmp_path / "bad.tlw"
    f.write_bytes(bytes(rec))
    lib = lin.load_library()
    assert lib.tl_weights_load(str(f).encode(), b"m") is None
    assert msg in lib.tl_last_error().decode()
    assert lib.tl_weights_cache_list(str(f).encode(), None, 0) == -1


def test_reader_reports_missing_record_and_file(lin, tmp_path):
    rng = np.random.default_rng(4)
    f = tmp_path / "w.tlw"
    f.write_bytes(fmt.record("a", *_w(rng, 16, 64)))
    lib = lin.load_library()
    assert lib.tl_weights_load(str(f).encode(), b"b") is None
    assert "no record named b" in lib.tl_last_error().decode()
    assert lib.tl_weights_load(str(tmp_path / "absent.tlw").encode(), b"a") is None
    assert "cannot open" in lib.tl_last_error().decode()
