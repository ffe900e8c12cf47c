"""tl_lm_head_argmax_noalloc_dev (the greedy step with the library's fixed
device work-space, for callers that cannot allocate) against
tl_lm_head_argmax_dev (its work-space allocated per stream): token, largest
logit and logits bit-exact on two calls in a row, the second smaller and on
the path whose final RMSNorm runs as its own launch into the work-space's
row buffer; an lm_head past the work-space's size is rejected."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
F = np.float32


def say(msg):
    print(f"[case] {msg}", flush=True)


def _case(lin, dev, rng, N, K):
    import torch
    w = torch.from_numpy(rng.integers(-127, 128, (N, K), dtype=np.int8)).to(dev)
    s = torch.from_numpy(rng.uniform(0.002, 0.02, N).astype(F)).to(dev)
    W = lin.DeviceWeights.from_codes(w, s)
    h = torch.from_numpy((rng.standard_normal(K) * 3).astype(F)).to(dev)
    nw = torch.from_numpy((1 + 0.1 * rng.standard_normal(K)).astype(F)).to(dev)
    return W, h, nw


def _run(fn, lin, dev, W, h, nw, N):
    import torch
    tok = torch.full((1,), -1, dtype=torch.int32, device=dev)
    mx = torch.full((1,), np.nan, dtype=torch.float32, device=dev)
    logits = torch.full((N,), np.nan, dtype=torch.float32, device=dev)
    fn(h, nw, W, tok, logits=logits, max_logit=mx)
    torch.cuda.synchronize()
    return int(tok.cpu()[0]), mx.cpu().numpy()[0], logits.cpu().numpy()


def test_lm_head_argmax_noalloc_equals_allocating_entry_point(lin, dev):
    rng = np.random.default_rng(355)
    for N, K in ((151936, 2048), (5000, 512)):       # second call smaller, norm as its own launch
        say(f"lm_head argmax no-alloc vs allocating N={N} K={K}")
        W, h, nw = _case(lin, dev, rng, N, K)
        want = _run(lin.lm_head_argmax_dev, lin, dev, W, h, nw, N)
        got = _run(lin.lm_head_argmax_noalloc_dev, lin, dev, W, h, nw, N)
        assert got[0] == want[0] and 0 <= got[0] < N
        assert got[1] == want[1] == want[2][want[0]]
        np.testing.assert_array_equal(got[2], want[2])
        assert int(np.argmax(got[2])) == got[0]
        W.close()


def test_lm_head_argmax_noalloc_rejects_oversize(lin, dev):
    import torch
    say("lm_head argmax no-alloc rejects 262160 rows")
    N, K = 262160, 128
    W = lin.DeviceWeights.from_codes(torch.ones((N, K), dtype=torch.int8, device=dev),
                                     torch.ones(N, dtype=torch.float32, device=dev))
    h = torch.ones(K, dtype=torch.float32, device=dev)
    tok = torch.zeros(1, dtype=torch.int32, device=dev)
    with pytest.raises(RuntimeError, match="no-allocation work-space"):
        lin.lm_head_argmax_noalloc_dev(h, None, W, tok)
    W.close()
