"""Device-pointer entry points called from several threads on one stream.

The library keeps one work-space (activation tiles, int8 planes, split
partials) per (device, stream) and grows it on demand.  Threads that enqueue
on the same stream (here the null stream, as callers who pass no stream do)
must take turns on it: a call that grows a buffer would otherwise free the
one another thread has just bound into its launches.  Four threads call
w8a8_linear_f32_dev and w8a32_linear_dev (the int8-plane path at these
batches) with batches of different sizes, so the buffers keep growing under
the other callers; every result must equal, bit for bit, the same call made
alone."""
import threading

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)


def test_shared_stream_threads_bit_identical(lin):
    import torch
    dev = torch.device("cuda:0")
    g = torch.Generator(device="cpu").manual_seed(5)
    N, K = 2048, 2048
    w = torch.randint(-127, 128, (N, K), dtype=torch.int8, generator=g)
    s = torch.rand(N, generator=g) * 0.018 + 0.002
    W = lin.DeviceWeights.from_codes(w.to(dev), s.to(dev))
    batches = [40, 200, 777, 1024]
    xs = [torch.randn((m, K), generator=g).to(dev) for m in batches]
    ops = [lin.w8a8_linear_f32_dev, lin.w8a32_linear_dev]
    want = {}
    for t, x in enumerate(xs):
        for o, op in enumerate(ops):
            y = torch.empty((x.shape[0], N), device=dev)
            op(x, W, y)
            torch.cuda.synchronize()
            want[t, o] = y.clone()
    say(f"4 threads x 12 rounds on the null stream, batches {batches}")
    errors = []

    def worker(t):
        try:
            ys = [torch.empty((xs[t].shape[0], N), device=dev) for _ in ops]
            for r in range(12):
                for o, op in enumerate(ops):
                    op(xs[t], W, ys[o])
                torch.cuda.synchronize()
                for o in range(len(ops)):
                    if not torch.equal(ys[o], want[t, o]):
                        errors.append((t, r, o))
        except Exception as e:  # reported by the main thread
            errors.append((t, repr(e)))

    ts = [threading.Thread(target=worker, args=(t,)) for t in range(len(xs))]
    for th in ts:
        th.start()
    for th in ts:
        th.join()
    W.close()
    assert not errors, errors[:8]
