"""The packed-weight cache file format written out independently of the
library, for the tests: the 16x64 lane-major k-block-major tile packing, the
64-byte record header and the four-lane streaming checksum.  A file built
here must load through tl_weights_load, and one written by tl_weights_save
must equal it byte for byte."""
import struct

import numpy as np

MAGIC = b"TLWCREC1"
VERSION = 1
HDR = struct.Struct("<8sII4iQQQQ")      # 64 bytes
M64 = (1 << 64) - 1


def pack_tiles(w: np.ndarray) -> bytes:
    """Tile (g, kb) at offset (kb*NG + g)*1024; byte b of lane l is
    W[16g + (l&15)][64kb + 16(l>>4) + b]; rows/cols past the matrix are 0."""
    rows, cols = w.shape
    NG, KB = -(-rows // 16), -(-cols // 64)
    p = np.zeros((NG * 16, KB * 64), np.int8)
    p[:rows, :cols] = w
    # [g, r, kb, j, b] -> [kb, g, j, r, b]   (lane = 16 j + r)
    t = p.reshape(NG, 16, KB, 4, 16).transpose(2, 0, 3, 1, 4)
    return np.ascontiguousarray(t).tobytes()


def padded_scales(s: np.ndarray) -> bytes:
    NG = -(-len(s) // 16)
    out = np.zeros(NG * 16, np.float32)
    out[:len(s)] = s
    return out.tobytes()


def _mix64(h, v):
    h ^= (v + 0x9E3779B97F4A7C15 + ((h << 6) & M64) + (h >> 2)) & M64
    h ^= h >> 31
    h = (h * 0xBF58476D1CE4E5B9) & M64
    return h ^ (h >> 29)


def _step(h, v):
    h = ((h ^ v) * 0x9E3779B97F4A7C15) & M64
    return h ^ (h >> 32)


def checksum(payload: bytes) -> int:
    """Four lanes over 32-byte blocks, lane j taking word j of each block
    (payloads here are whole blocks: tiles are 1 KiB, scales 64 B per group)."""
    assert len(payload) % 32 == 0
    h = [0x243F6A8885A308D3, 0x13198A2E03707344, 0xA4093822299F31D0, 0x082EFA98EC4E6C89]
    words = np.frombuffer(payload, dtype="<u8").reshape(-1, 4)
    for row in words.tolist():
        for j in range(4):
            h[j] = _step(h[j], row[j])
    v = len(payload)
    for j in range(4):
        v = _mix64(v, h[j])
    return v


def record(name: str, w: np.ndarray, s: np.ndarray, corrupt: bool = False) -> bytes:
    rows, cols = w.shape
    NG, KB = -(-rows // 16), -(-cols // 64)
    tiles, scales = pack_tiles(w), padded_scales(s)
    nb = name.encode()
    hdr = HDR.pack(MAGIC, VERSION, len(nb), rows, cols, NG, KB, len(tiles), len(scales),
                   checksum(tiles + scales), 0)
    body = tiles + scales
    if corrupt:
        body = bytearray(body)
        body[len(body) // 3] ^= 0x40
        body = bytes(body)
    return hdr + nb + b"\0" * (-len(nb) % 64) + body
