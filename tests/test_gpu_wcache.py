"""GPU checks of the packed-weight cache file and of the quantize-and-pack
load step (survey row f-3; reference load path decoder.py:248-317 and
kernel/w8a32_kernel.c:63-108).

Bars: files written by tl_weights_save equal, byte for byte, the format
restated in tests/wcache_format.py; loaded matrices export the exact codes
and scales and give bit-identical GEMV outputs; damaged payloads are
rejected; w8a32_quantize leaves the packed matrix in the registry, so the
first linear call on its host arrays uploads nothing."""
import numpy as np
import pytest

import wcache_format as fmt

pytestmark = pytest.mark.gpu
F = np.float32


def say(msg):
    print(f"[case] {msg}", flush=True)


def _w(rng, rows, cols):
    return rng.integers(-127, 128, (rows, cols), dtype=np.int8), rng.uniform(0.002, 0.02, rows).astype(F)


def test_save_load_round_trip(lin, orc, dev, tmp_path):
    import torch
    say("weight cache save/load round trip")
    rng = np.random.default_rng(10)
    mats = {"layers.0.o_proj": _w(rng, 300, 1000), "layers.3.gate_up_proj": _w(rng, 4096, 2048),
            "lm_head": _w(rng, 37, 70)}
    path = tmp_path / "w.tlw"
    for i, (name, (w, s)) in enumerate(mats.items()):
        W = lin.DeviceWeights.from_codes(w, s)
        W.save(str(path), name, append=i > 0)
        W.close()
    assert lin.cache_list(str(path)) == list(mats)
    assert path.read_bytes() == b"".join(fmt.record(n, w, s) for n, (w, s) in mats.items())
    for name, (w, s) in reversed(list(mats.items())):
        L = lin.DeviceWeights.load(str(path), name)
        codes, scales = L.export()
        np.testing.assert_array_equal(codes, w)
        np.testing.assert_array_equal(scales, s)
        x = rng.standard_normal((1, w.shape[1])).astype(F)
        y = torch.empty((1, w.shape[0]), dtype=torch.float32, device=dev)
        lin.w8a32_linear_dev(torch.from_numpy(x).to(dev), L, y)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(y.cpu().numpy(), orc.w8a32_linear(x, w, s))
        L.close()
    # replace (append=False) leaves one record
    W = lin.DeviceWeights.from_codes(*mats["lm_head"])
    W.save(str(path), "only", append=False)
    W.close()
    assert lin.cache_list(str(path)) == ["only"]


def test_file_built_from_format_loads(lin, tmp_path):
    say("weight cache from the restated format")
    rng = np.random.default_rng(11)
    w, s = _w(rng, 129, 333)
    path = tmp_path / "py.tlw"
    path.write_bytes(fmt.record("x", *_w(rng, 16, 64)) + fmt.record("m", w, s))
    L = lin.DeviceWeights.load(str(path), "m")
    codes, scales = L.export()
    L.close()
    np.testing.assert_array_equal(codes, w)
    np.testing.assert_array_equal(scales, s)


def test_damaged_payload_rejected(lin, tmp_path):
    say("weight cache checksum mismatch")
    rng = np.random.default_rng(12)
    path = tmp_path / "bad.tlw"
    path.write_bytes(fmt.record("m", *_w(rng, 64, 256), corrupt=True))
    lib = lin.load_library()
    assert lib.tl_weights_load(str(path).encode(), b"m") is None
    assert "checksum mismatch" in lib.tl_last_error().decode()


def test_quantize_packs_into_registry(lin, orc):
    """w8a32_quantize (host pointers) quantizes and packs in one pass; the
    registry then already holds the matrix for the returned arrays."""
    say("quantize-and-pack registry entry")
    lib = lin.load_library()
    lib.tl_registry_clear()
    rng = np.random.default_rng(13)
    wf = (rng.standard_normal((1000, 2048)) * 0.02).astype(F)
    q, s = lin.quantize(wf)
    want_q, want_s = orc.quantize_rows(wf)
    np.testing.assert_array_equal(q, want_q)
    np.testing.assert_array_equal(s, want_s)
    assert lib.tl_registry_entries() == 1
    nbytes = lib.tl_registry_bytes()
    assert nbytes == 63 * 32 * 1024 + 63 * 16 * 4
    x = rng.standard_normal((1, 2048)).astype(F)
    np.testing.assert_array_equal(lin.w8a32_linear(x, q, s), orc.w8a32_linear(x, q, s))
    xb = rng.standard_normal((5, 2048)).astype(F)
    y5 = lin.w8a32_linear(xb, q, s)
    assert np.linalg.norm(y5 - orc.w8a32_linear(xb, q, s)) <= 1e-5 * np.linalg.norm(y5)
    assert lib.tl_registry_entries() == 1 and lib.tl_registry_bytes() == nbytes
    # changing the host codes in place is still detected (fingerprint)
    q[:, :] = -q
    np.testing.assert_array_equal(lin.w8a32_linear(x, q, s), orc.w8a32_linear(x, q, s))
    lib.tl_registry_clear()


def test_decoder_cache_round_trip(lin, tmp_path):
    """Decoder.save_cache then Decoder.from_cache: every projection and the
    greedy token agree bit for bit, and loading uploads nothing beyond the
    records (the registry holds exactly the loaded matrices)."""
    from typhoon_ocr_server_amd import decoder as dec
    say("decoder cache round trip")
    lib = lin.load_library()
    lib.tl_registry_clear()
    rng = np.random.default_rng(14)
    K, V = 2048, 32768
    layers = [dec.random_layer_weights(rng) for _ in range(2)]
    lm = (rng.standard_normal((V, K)) * 0.02).astype(F)
    nw = (1.0 + 0.1 * rng.standard_normal(K)).astype(F)
    d = dec.Decoder(layers, lm_head=lm, final_norm=nw)
    path = tmp_path / "decoder.tlw"
    d.save_cache(str(path))
    names = lin.cache_list(str(path))
    assert len(names) == 2 * 9 + 1 and names[-1] == "lm_head"
    lib.tl_registry_clear()
    d2 = dec.Decoder.from_cache(str(path), final_norm=nw)
    assert lib.tl_registry_entries() == len(names)
    reg_bytes = lib.tl_registry_bytes()
    for l_idx in range(2):
        for name in dec.PROJECTIONS + ("qkv_proj", "gate_up_proj"):
            w, s = d.layers[l_idx][name]
            w2, s2 = d2.layers[l_idx][name]
            np.testing.assert_array_equal(w2, w)
            np.testing.assert_array_equal(s2, s)
            x = rng.standard_normal((1, w.shape[1])).astype(F)
            np.testing.assert_array_equal(d2.project(l_idx, name, x), d.project(l_idx, name, x))
    for _ in range(3):
        hs = (rng.standard_normal((2, K)) * 4).astype(F)
        assert d2.next_token(hs) == d.next_token(hs)
        np.testing.assert_array_equal(d2.get_logits(hs), d.get_logits(hs))
    assert lib.tl_registry_bytes() >= reg_bytes
    lib.tl_registry_clear()
