"""The host-pointer ABI (w8a32_linear, w8a16_linear: host arrays in and out,
weights through the registry) is reentrant across caller threads, as the
reference's functions are (kernel/w8a32_kernel.c:355-370: plain functions
over caller-owned arrays): each call leases its own stream and staging
buffers, and registry entries are shared with the calls using them.

Eight threads call the ABI at once on their own weights, while another
thread keeps clearing and evicting the registry (forcing re-uploads under the
callers' feet); every result must equal, bit for bit, the same call made
alone.  A second check times the same work from 1 and from 4 threads."""
import threading
import time

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
F = np.float32


def say(msg):
    print(f"[case] {msg}", flush=True)


def _bf16_bits(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _cases(rng, n):
    shapes = [(2048, 2048), (4096, 2048), (300, 1000), (2048, 6144)]
    out = []
    for t in range(n):
        N, K = shapes[t % len(shapes)]
        x = rng.standard_normal((4, K)).astype(F)
        w = rng.integers(-127, 128, (N, K), dtype=np.int8)
        s = (rng.random(N) * 0.018 + 0.002).astype(F)
        b = rng.standard_normal(N).astype(F)
        out.append((x, w, s, b))
    return out


def _run(lin, case):
    x, w, s, b = case
    return [lin.w8a32_linear(np.ascontiguousarray(x[:1]), w, s, bias=b), lin.w8a32_linear(x, w, s),
            lin.w8a16_linear(_bf16_bits(x[:1]), w, s, bias=b), lin.w8a16_linear(_bf16_bits(x), w, s)]


def test_host_abi_threads_bit_identical(lin):
    say("host ABI: 8 threads x 10 rounds against calls made alone, registry cleared meanwhile")
    lib = lin.load_library()
    cases = _cases(np.random.default_rng(11), 8)
    want = [_run(lin, c) for c in cases]
    errors = []
    stop = threading.Event()

    def worker(i):
        try:
            for _ in range(10):
                for g, wnt in zip(_run(lin, cases[i]), want[i]):
                    np.testing.assert_array_equal(g, wnt)
        except Exception as e:  # reported by the main thread
            errors.append((i, repr(e)))

    def evictor():
        k = 0
        while not stop.is_set():
            if k % 2:
                lib.tl_registry_clear()
            else:
                lib.tl_evict_weights(cases[k % len(cases)][1].ctypes.data_as(lin._i8p))
            k += 1
            time.sleep(0.002)

    ev = threading.Thread(target=evictor)
    ts = [threading.Thread(target=worker, args=(i,)) for i in range(len(cases))]
    ev.start()
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=300)
    stop.set()
    ev.join(timeout=60)
    assert not any(t.is_alive() for t in ts)
    assert not errors, errors[:3]
    lib.tl_registry_clear()


def test_host_abi_threads_overlap(lin):
    """Four threads of batch-1 w8a32_linear calls on resident weights (one
    ctypes call each, which releases the interpreter lock) finish 4000 calls
    in well under the time one thread takes for them: the calls overlap
    (each on its own leased stream) instead of queueing on a lock.  Measured
    18.6 us per call alone against 6.4 us per call from four threads."""
    say("host ABI: 1 vs 4 threads")
    lib = lin.load_library()
    rng = np.random.default_rng(12)
    calls = []
    keep = []
    for _ in range(4):
        N, K = 4096, 2048
        x = rng.standard_normal((1, K)).astype(F)
        w = rng.integers(-127, 128, (N, K), dtype=np.int8)
        s = (rng.random(N) * 0.018 + 0.002).astype(F)
        y = np.empty((1, N), F)
        keep.append((x, w, s, y))
        calls.append((x.ctypes.data_as(lin._f32p), w.ctypes.data_as(lin._i8p), s.ctypes.data_as(lin._f32p),
                      y.ctypes.data_as(lin._f32p), N, K))
    fn = lib.w8a32_linear

    def work(c, n):
        xp, wp, sp, yp, N, K = c
        for _ in range(n):
            fn(xp, wp, sp, None, yp, None, 1, N, K)

    for c in calls:
        work(c, 5)                                  # weights resident, contexts made
    n = 1000
    t0 = time.perf_counter()
    for c in calls:
        work(c, n)
    t_one = time.perf_counter() - t0
    ts = [threading.Thread(target=work, args=(c, n)) for c in calls]
    t0 = time.perf_counter()
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=300)
    t_four = time.perf_counter() - t0
    say(f"1 thread {t_one * 1e6 / (4 * n):.1f} us/call, 4 threads {t_four * 1e6 / (4 * n):.1f} us/call")
    assert lib.tl_last_error() is None
    assert t_four < 0.7 * t_one, (t_one, t_four)
