"""GPU parity of the fused greedy step: final RMSNorm + lm_head GEMV + argmax
(reference decoder.py:443-464, _get_logits and the greedy branch of _sample).

Bars: the normalised row bit-exact against numpy's own float32 expression
(the reference computes it with numpy); logits bit-exact against the
oracle's w8a32_linear on that row; the token equal to the first index of the
largest logit (torch.argmax's rule, np.argmax's too).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
F = np.float32


def say(msg):
    print(f"[case] {msg}", flush=True)


def np_final_norm(h, w):
    """The reference's expression, decoder.py:444-446, in numpy float32."""
    rms = np.sqrt(np.mean(h * h) + 1e-6)
    return (h / rms) * w if w is not None else h / rms


@pytest.mark.parametrize("K", [128, 1024, 2048, 4096, 16384])
@pytest.mark.parametrize("scale", [1e-3, 1.0, 37.5])
def test_rmsnorm_matches_numpy(lin, dev, K, scale):
    import torch
    say(f"rmsnorm K={K} scale={scale}")
    rng = np.random.default_rng(K + int(scale * 10))
    h = (rng.standard_normal(K) * scale).astype(F)
    w = (1.0 + 0.1 * rng.standard_normal(K)).astype(F)
    for wv in (w, None):
        out = torch.empty(K, dtype=torch.float32, device=dev)
        lin.rmsnorm_np_dev(torch.from_numpy(h).to(dev), None if wv is None else torch.from_numpy(wv).to(dev), out)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy(), np_final_norm(h, wv))


def _check_step(lin, orc, dev, h, nw, W, w, s):
    import torch
    N = w.shape[0]
    want_logits = orc.w8a32_linear(np_final_norm(h, nw)[None], w, s)[0]
    tok = torch.full((1,), -1, dtype=torch.int32, device=dev)
    logits = torch.empty(N, dtype=torch.float32, device=dev)
    mx = torch.empty(1, dtype=torch.float32, device=dev)
    lin.lm_head_argmax_dev(torch.from_numpy(h).to(dev), torch.from_numpy(nw).to(dev), W, tok, logits, mx)
    torch.cuda.synchronize()
    got = logits.cpu().numpy()
    np.testing.assert_array_equal(got, want_logits)
    t = int(tok.cpu().numpy()[0])
    assert t == int(np.argmax(want_logits)), (t, int(np.argmax(want_logits)))
    assert mx.cpu().numpy()[0] == want_logits[t]
    # without a logits buffer the token is the same
    tok2 = torch.full((1,), -1, dtype=torch.int32, device=dev)
    lin.lm_head_argmax_dev(torch.from_numpy(h).to(dev), torch.from_numpy(nw).to(dev), W, tok2)
    torch.cuda.synchronize()
    assert int(tok2.cpu().numpy()[0]) == t
    return t


@pytest.mark.parametrize("N,K", [(151936, 2048), (1000, 2048), (4100, 1024), (37, 128)])
def test_lm_head_argmax_dev(lin, orc, dev, N, K):
    say(f"lm_head argmax N={N} K={K}")
    rng = np.random.default_rng(N + K)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    s = rng.uniform(0.002, 0.02, N).astype(F)
    nw = (1.0 + 0.1 * rng.standard_normal(K)).astype(F)
    W = lin.DeviceWeights.from_codes(w, s)
    for i in range(4 if N > 100000 else 6):
        h = (rng.standard_normal(K) * rng.uniform(0.5, 20)).astype(F)
        _check_step(lin, orc, dev, h, nw, W, w, s)
    W.close()


def test_lm_head_argmax_ties_take_lowest_index(lin, orc, dev):
    """Identical rows give identical logits; the largest of them must be
    reported at its lowest index, across work-groups and within one."""
    say("lm_head argmax ties")
    rng = np.random.default_rng(7)
    N, K = 6000, 2048
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    s = rng.uniform(0.002, 0.02, N).astype(F)
    h = rng.standard_normal(K).astype(F)
    nw = np.ones(K, F)
    x = np_final_norm(h, nw)
    # row 4321 is the best row of a random set; copy it to 5999, 1234 and 1235
    best = np.sign(x).astype(np.int8) * 120
    w[4321] = best
    s[4321] = 0.05
    for r in (5999, 1234, 1235):
        w[r] = best
        s[r] = 0.05
    W = lin.DeviceWeights.from_codes(w, s)
    t = _check_step(lin, orc, dev, h, nw, W, w, s)
    assert t == 1234
    W.close()


def test_host_lm_head_argmax_and_decoder_next_token(lin, orc):
    """tl_lm_head_argmax on host pointers, and Decoder.next_token, equal the
    reference's two steps (get_logits, then the greedy argmax)."""
    from typhoon_ocr_server_amd import decoder as dec
    say("host lm_head argmax + Decoder.next_token")
    rng = np.random.default_rng(11)
    K, V = 2048, 32768
    lm = (rng.standard_normal((V, K)) * 0.02).astype(F)
    nw = (1.0 + 0.1 * rng.standard_normal(K)).astype(F)
    layer = dec.random_layer_weights(rng)
    d = dec.Decoder([layer], lm_head=lm, final_norm=nw)
    for i in range(5):
        hs = (rng.standard_normal((3, K)) * 4).astype(F)
        want = d.sample(d.get_logits(hs))
        assert d.next_token(hs) == want
        logits = np.empty(V, F)
        t = lin.lm_head_argmax(hs[-1], nw, d._lm_head_w, d._lm_head_s, logits)
        assert t == want
        np.testing.assert_array_equal(logits, d.get_logits(hs))
