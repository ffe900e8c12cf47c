"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Checks: golden vectors computed independently (tests/golden/make_golden.py),
closed forms and invariants of the quantizer, brute-force integer dots,
float64 brute force for the dequant-then-SGEMM branch, linearity.  Each check
is chosen so that a plausible mistake fails it (see the comments).
"""
import numpy as np
import pytest

F = np.float32


def _split(flat, lens):
    out, o = [], 0
    for n in lens:
        out.append(flat[o:o + n]); o += n
    return out


@pytest.mark.parametrize("clamp", [1, 0])
def test_quantizer_golden(orc, golden, clamp):
    srcs = _split(golden["quant_src"], golden["quant_len"])
    codes = _split(golden[f"quant_codes_c{clamp}"], golden["quant_len"])
    for i, (src, want) in enumerate(zip(srcs, codes)):
        q, s = orc.quantize_rows(src, clamp_main=bool(clamp))
        assert s[0] == golden[f"quant_scales_c{clamp}"][i], i
        np.testing.assert_array_equal(q[0], want, err_msg=f"case {i}")


def test_quantizer_closed_forms(orc):
    rng = np.random.default_rng(7)
    for K in (16, 48, 2048, 6144, 37, 1):
        x = (rng.standard_normal((5, K)) * rng.uniform(1e-3, 1e3, (5, 1))).astype(F)
        q, s = orc.quantize_rows(x)
        for r in range(5):
            absmax = np.max(np.abs(x[r]))
            assert s[r] == F(absmax) / F(127)                       # scale formula
            assert np.all(np.abs(q[r].astype(int)) <= 127)
            j = int(np.argmax(np.abs(x[r])))
            assert abs(int(q[r, j])) == 127                          # argmax -> +-127
            err = np.abs(x[r].astype(np.float64) - q[r].astype(np.float64) * float(s[r]))
            # round-to-nearest: truncation or floor would break this bound
            assert np.all(err <= float(s[r]) / 2 * (1 + 2.0 ** -22)), K


def test_quantizer_ties(orc):
    # s == 1 exactly (absmax 127): vector region rounds ties to even ...
    x = np.zeros(32, F); x[0] = 127
    x[1:7] = [2.5, 3.5, -2.5, -3.5, 0.5, -0.5]
    q, s = orc.quantize_rows(x)
    assert s[0] == 1.0
    assert list(q[0, 1:7]) == [2, 4, -2, -4, 0, 0]
    # ... and the scalar tail (k >= K & ~15) rounds ties away from zero (lroundf)
    x = np.zeros(21, F); x[0] = 127
    x[16:21] = [2.5, -2.5, 0.5, -0.5, 3.5]
    q, _ = orc.quantize_rows(x)
    assert list(q[0, 16:21]) == [3, -3, 1, -1, 4]


def test_quantizer_uses_reciprocal_multiply(orc):
    # code = rne(fl(x * fl(1/s))), not rne(fl(x / s)): find rows where the
    # two differ (vectorised search) and require the first.
    rng = np.random.default_rng(11)
    x = rng.standard_normal((400000, 16)).astype(F)
    s = np.max(np.abs(x), axis=1) / F(127)
    inv = F(1) / s
    a = np.rint(x * inv[:, None])
    b = np.rint(x / s[:, None])
    rows = np.nonzero(np.any(a != b, axis=1))[0][:64]
    assert rows.size > 0
    q, qs = orc.quantize_rows(x[rows])
    np.testing.assert_array_equal(qs, s[rows])
    np.testing.assert_array_equal(q, a[rows].astype(np.int8))


def test_quantizer_special_rows(orc):
    q, s = orc.quantize_rows(np.zeros((2, 40), F))
    assert np.all(s == 1.0) and np.all(q == 0)
    # NaN in the 16-aligned prefix: absmax is NaN, `absmax > 0` is false, s = 1
    x = np.linspace(-3, 3, 32).astype(F); x[5] = np.nan
    q, s = orc.quantize_rows(x)
    assert s[0] == 1.0 and q[0, 5] == 0 and q[0, 31] == 3
    # NaN only in the scalar tail is ignored by the `v > absmax` scan
    x = np.linspace(-3, 3, 20).astype(F); x[18] = np.nan
    q, s = orc.quantize_rows(x)
    assert s[0] == F(3) / F(127) and q[0, 18] == 0
    # Inf: scale Inf, inv 0, every code 0
    x = np.ones(16, F); x[2] = np.inf
    q, s = orc.quantize_rows(x)
    assert np.isinf(s[0]) and np.all(q == 0)


def _arm_fcvtas_x(v: float) -> int:
    """FCVTAS Xd, Sn per the Arm ARM (FPToFixed, rounding FPRounding_TIEAWAY,
    64-bit signed destination): NaN -> 0, round half away from zero,
    saturate to [-2^63, 2^63 - 1]."""
    import math
    if math.isnan(v):
        return 0
    if math.isinf(v):
        return 2 ** 63 - 1 if v > 0 else -(2 ** 63)
    r = math.floor(abs(v) + 0.5) * (1 if v >= 0 else -1)
    return max(-(2 ** 63), min(2 ** 63 - 1, r))


def _low32(r: int) -> int:
    """C's conversion of a 64-bit integer to int on clang/AArch64: the low 32
    bits, two's complement."""
    u = r & 0xFFFFFFFF
    return u - 2 ** 32 if u >= 2 ** 31 else u


@pytest.mark.parametrize("clamp", [True, False])
def test_quantizer_tail_overflowing_reciprocal(orc, clamp):
    """absmax so small that fl(absmax/127) rounds to 0: inv = +inf.  The
    16-aligned prefix saturates (FCVTNS, SQXTN: +inf -> 127, -inf -> -128,
    clamped to -127 by the weight quantizers, NaN = 0*inf -> 0); the scalar
    tail evaluates (int)lroundf(x*inv), which the reference's AArch64 build
    computes as FCVTAS into a 64-bit register, keeping the low 32 bits, then
    clamps to [-127, 127].  Expected codes come from the Arm definition
    (_arm_fcvtas_x); glibc's lroundf (+inf -> 0) or a 32-bit FCVTAS
    (+inf -> 127) would fail the positive tail elements."""
    x = np.array([1.4e-45, -2.8e-45, 0.0, 4.2e-45] * 4 + [2.8e-45, -1.4e-45, 0.0, 4.2e-45, -4.2e-45], F)
    assert x[0] > 0 and x[1] < 0                       # denormals, not flushed
    q, s = orc.quantize_rows(x, clamp_main=clamp)
    assert s[0] == F(np.abs(x).max()) / F(127) == 0.0
    inv = F(1) / s[0] if s[0] != 0 else np.float32(np.inf)
    want = []
    for k, v in enumerate(x):
        with np.errstate(invalid="ignore", over="ignore"):
            p = float(np.float32(v) * inv)
        if k < 16:
            c = 0 if np.isnan(p) else (127 if p > 0 else (-127 if clamp else -128))
        else:
            c = min(127, max(-127, _low32(_arm_fcvtas_x(p))))
        want.append(c)
    assert want[16:] == [-1, 0, 0, -1, 0]
    assert list(q[0]) == want


def test_activation_quantizer_matches_weight_quantizer(orc):
    # |x*inv| <= 127 (1 + 3 eps) always rounds into [-127, 127], so the
    # missing clamp of the activation quantizer never changes a code.
    rng = np.random.default_rng(3)
    x = rng.standard_normal((64, 2048)).astype(F)
    a, sa = orc.quantize_rows(x, clamp_main=False)
    b, sb = orc.quantize_rows(x, clamp_main=True)
    np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(sa, sb)


def test_int_acc_bruteforce(orc):
    rng = np.random.default_rng(5)
    xq = rng.integers(-127, 128, (3, 70), dtype=np.int8)
    w = rng.integers(-127, 128, (9, 70), dtype=np.int8)
    acc = orc.int_acc(xq, w)
    for b in range(3):
        for n in range(9):
            assert acc[b, n] == sum(int(i) * int(j) for i, j in zip(xq[b], w[n]))
    # the largest |acc| the reference can produce at K = 6144 still fits int32
    xq = np.full((1, 6144), -127, np.int8)
    w = np.full((2, 6144), -127, np.int8)
    assert orc.int_acc(xq, w)[0, 0] == 127 * 127 * 6144


@pytest.mark.parametrize("tag", ["a", "b", "c"])
def test_gemv_golden(orc, golden, tag):
    g = {k[len(f"gemv_{tag}_"):]: v for k, v in golden.items() if k.startswith(f"gemv_{tag}_")}
    y, codes, xs, acc = orc.w8a32_linear(g["x"][None], g["w"], g["ws"], detail=True)
    np.testing.assert_array_equal(codes, g["codes"])
    assert xs == g["xs"][0]
    np.testing.assert_array_equal(acc, g["acc"])
    np.testing.assert_array_equal(y[0], g["y"])                       # bit-exact
    yb = orc.w8a32_linear(g["x"][None], g["w"], g["ws"], bias=g["bias"])
    np.testing.assert_array_equal(yb[0], g["ybias"])
    y8 = orc.w8a8_linear(codes[None], g["xs"], g["w"], g["ws"], bias=g["bias"])
    np.testing.assert_array_equal(y8[0], g["y8bias"])                 # fused epilogue


@pytest.mark.parametrize("threads", [1, 3, 8])
@pytest.mark.parametrize("N,K", [(6144, 2048), (2048, 6144), (37, 50), (1000, 1021)])
def test_cpu_baseline_gemv_equals_oracle(orc, N, K, threads):
    """The timed CPU-baseline GEMV (orc_w8a32_gemv_timed: the reference's
    row-chunk fan-out) computes exactly orc_w8a32_linear at batch 1, for any
    thread count, in both builds (x86-64-v3 and -march=native), so the GB/s
    it reports are for the reference's arithmetic."""
    rng = np.random.default_rng(N + K + threads)
    x = rng.standard_normal((1, K)).astype(F)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    s = rng.uniform(0.002, 0.02, N).astype(F)
    want = orc.w8a32_linear(x, w, s)[0]
    for native in (False, True):
        y = np.full(N, np.nan, F)
        orc.w8a32_gemv_timed(x, w, s, y, threads, native=native)
        np.testing.assert_array_equal(y, want)


def test_gemv_epilogue_order(orc):
    # fl(fl(acc*ws)*xs) and fl(acc*fl(ws*xs)) differ in many outputs; the
    # oracle must produce the first (w8a32_kernel.c:239).
    rng = np.random.default_rng(1234)
    N, K = 6144, 2048
    x = rng.standard_normal(K).astype(F)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    ws = rng.uniform(0.002, 0.02, N).astype(F)
    y, codes, xs, acc = orc.w8a32_linear(x[None], w, ws, detail=True)
    want = (acc.astype(F) * ws) * F(xs)
    other = acc.astype(F) * (ws * F(xs))
    np.testing.assert_array_equal(y[0], want)
    assert np.count_nonzero(want != other) > 100


def test_gemm_golden_and_bruteforce(orc, golden):
    X, w, ws, Y = golden["gemm_X"], golden["gemm_w"], golden["gemm_ws"], golden["gemm_Y"]
    y = orc.w8a32_linear(X, w, ws)
    np.testing.assert_allclose(y, Y, rtol=1e-6, atol=1e-6)
    # float64 brute force of dequant-then-dot on a larger case
    rng = np.random.default_rng(9)
    M, N, K = 5, 64, 2048
    X = rng.standard_normal((M, K)).astype(F)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    ws = rng.uniform(0.002, 0.02, N).astype(F)
    wd = (w.astype(F) * ws[:, None]).astype(np.float64)
    want = (X.astype(np.float64) @ wd.T).astype(F)
    y = orc.w8a32_linear(X, w, ws)
    rel = np.linalg.norm(y - want) / np.linalg.norm(want)
    assert rel < 1e-7
    # linearity in X (a dropped or transposed term breaks it)
    y2 = orc.w8a32_linear(2 * X, w, ws)
    np.testing.assert_allclose(y2, 2 * y, rtol=1e-6, atol=1e-6)


def test_gemm_bias_is_separate_rounding(orc):
    rng = np.random.default_rng(2)
    M, N, K = 2, 16, 64
    X = rng.standard_normal((M, K)).astype(F)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    ws = rng.uniform(0.002, 0.02, N).astype(F)
    b = rng.standard_normal(N).astype(F)
    np.testing.assert_array_equal(orc.w8a32_linear(X, w, ws, bias=b),
                                  orc.w8a32_linear(X, w, ws) + b)


def test_w8a8_batch_paths(orc):
    rng = np.random.default_rng(4)
    M, N, K = 4, 48, 256
    X = rng.standard_normal((M, K)).astype(F)
    xq, xs = orc.quantize_rows(X)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    ws = rng.uniform(0.002, 0.02, N).astype(F)
    y = orc.w8a8_linear(xq, xs, w, ws)
    acc = orc.int_acc(xq, w).astype(np.float64)
    exact = acc * ws.astype(np.float64)[None] * xs.astype(np.float64)[:, None]
    assert np.linalg.norm(y - exact) / np.linalg.norm(exact) < 1e-6
    # batch == 1 row equals the M=1 epilogue on the same codes
    y1 = orc.w8a8_linear(xq[:1], xs[:1], w, ws)
    want = (acc[0].astype(F) * ws) * xs[0]
    np.testing.assert_array_equal(y1[0], want.astype(F))


def test_w8a16_paths(orc):
    rng = np.random.default_rng(6)
    M, N, K = 3, 32, 264
    X = rng.standard_normal((M, K)).astype(F)
    xb = (X.view(np.uint32) + 0x7fff + ((X.view(np.uint32) >> 16) & 1)) >> 16
    xb = xb.astype(np.uint16)
    xf = (xb.astype(np.uint32) << 16).view(F).astype(np.float64)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    ws = rng.uniform(0.002, 0.02, N).astype(F)
    for m in (1, M):
        y = orc.w8a16_linear(xb[:m], w, ws)
        exact = (xf[:m] @ w.astype(np.float64).T) * ws.astype(np.float64)
        assert np.linalg.norm(y - exact) / np.linalg.norm(exact) < 1e-6


def test_nonfinite_rows_closed_form(orc):
    """A token row holding +Inf at column kp and -Inf at column kn: the
    reference's fp32 sums of x times the dequantized weights (scales > 0) give,
    output by output, IEEE's closed form: NaN where a weight code at kp or kn
    is 0 (inf * 0) or where sign(w[n,kp]) != -sign(w[n,kn]) (inf - inf), else
    that common sign times Inf; finite terms change nothing.  A NaN anywhere
    in the row gives NaN everywhere.  Checked on the W8A32 batch branch
    (dequantize then SGEMM) and the W8A16 bf16 branch at 1 and 3 tokens; a
    summation that dropped the Inf terms, or took the code's magnitude for its
    sign, fails it."""
    rng = np.random.default_rng(17)
    M, N, K = 3, 96, 264
    kp, kn = 9, 200
    x = rng.standard_normal((M, K)).astype(F)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    w[::7, kp] = 0
    w[3::11, kn] = 0
    ws = rng.uniform(0.002, 0.02, N).astype(F)
    x[1, kp], x[1, kn] = np.inf, -np.inf
    x[2, 40] = np.nan
    sp, sn = np.sign(w[:, kp].astype(int)), -np.sign(w[:, kn].astype(int))
    want = np.where((sp == 0) | (sn == 0) | (sp != sn), np.nan, np.where(sp > 0, np.inf, -np.inf))
    assert np.isnan(want).any() and np.isposinf(want).any() and np.isneginf(want).any()
    y = orc.w8a32_linear(x, w, ws, bias=rng.standard_normal(N).astype(F))
    np.testing.assert_array_equal(y[1], want)
    assert np.isnan(y[2]).all() and np.isfinite(y[0]).all()
    xb = ((x.view(np.uint32).astype(np.uint64) + 0x7fff + ((x.view(np.uint32) >> 16) & 1)) >> 16).astype(np.uint16)
    np.testing.assert_array_equal(orc.w8a16_linear(xb, w, ws)[1], want)
    np.testing.assert_array_equal(orc.w8a16_linear(xb[1:2], w, ws)[0], want)


def _pairwise_model(x):
    """The summation order the GPU final-RMSNorm kernel uses for K = 128*2^j:
    per 128-block 8 interleaved accumulators, ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)),
    then a balanced tree over the blocks (float32 throughout)."""
    f = np.float32
    nb = len(x) // 128
    blk = []
    for b in range(nb):
        r = []
        for j in range(8):
            acc = f(x[128 * b + j] * x[128 * b + j])
            for i in range(1, 16):
                v = x[128 * b + 8 * i + j]
                acc = f(acc + f(v * v))
            r.append(acc)
        blk.append(f(f(f(r[0] + r[1]) + f(r[2] + r[3])) + f(f(r[4] + r[5]) + f(r[6] + r[7]))))
    w = 1
    while w < nb:
        for i in range(0, nb, 2 * w):
            blk[i] = f(blk[i] + blk[i + w])
        w *= 2
    return blk[0]


@pytest.mark.parametrize("K", [128, 256, 1024, 2048, 4096])
def test_numpy_mean_order_matches_kernel_model(K):
    """decoder.py:444 computes np.mean(h * h) in float32; numpy sums with its
    pairwise algorithm.  The GPU kernel follows the model above; this pins
    that the installed numpy sums in exactly that order (and divides by K in
    float32), on vectors of very different scales."""
    rng = np.random.default_rng(K)
    for t in range(40):
        h = (rng.standard_normal(K) * 10.0 ** rng.uniform(-4, 4)).astype(np.float32)
        s = _pairwise_model(h)
        assert s == np.add.reduce((h * h).astype(np.float32))
        assert np.mean(h * h) == np.float32(s / np.float32(K))


@pytest.mark.parametrize("M,N,K", [(2, 130, 70), (37, 300, 257), (64, 256, 2048)])
def test_cpu_baseline_gemms_match_checker(orc, M, N, K):
    """The timed CPU-baseline legs (the reference's tile decompositions on a
    blocked fp32 SGEMM) compute what the pinned checker computes: W8A32 and
    W8A8 batch > 1 and W8A16 (batch 1 and > 1) within relative L2 1e-5 of
    the float64-accumulated oracle, with and without bias, in both builds;
    ragged shapes exercise the tile and register-block edges."""
    rng = np.random.default_rng(M * 7 + N + K)
    x = rng.standard_normal((M, K)).astype(F)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    s = rng.uniform(0.002, 0.02, N).astype(F)
    b = rng.standard_normal(N).astype(F)
    xq, xs = orc.quantize_rows(x)
    u = x.view(np.uint32).astype(np.uint64)
    xb = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)

    def rel(a, r):
        return float(np.linalg.norm(a.astype(np.float64) - r) / np.linalg.norm(r))
    for native in (False, True):
        for bias in (None, b):
            assert rel(orc.base_w8a32_gemm(x, w, s, 3, native, bias), orc.w8a32_linear(x, w, s, bias=bias)) <= 1e-5
            assert rel(orc.base_w8a8_gemm(xq, xs, w, s, 3, native, bias),
                       orc.w8a8_linear(xq, xs, w, s, bias=bias)) <= 1e-5
            assert rel(orc.base_w8a16_linear(xb, w, s, 3, native, bias), orc.w8a16_linear(xb, w, s, bias=bias)) <= 1e-5
            assert rel(orc.base_w8a16_linear(xb[:1], w, s, 3, native, bias),
                       orc.w8a16_linear(xb[:1], w, s, bias=bias)) <= 1e-5


def test_frecpe_quotient_from_any_faithful_reciprocal():
    """The device restatement of FRECPE takes floor(2^19 / a), for the odd
    a = 2 (256 + m) + 1 in [513, 1023] that the estimate's eight mantissa
    bits give, as trunc(2^19 * rcp(a)) with the hardware reciprocal, which is
    within one ulp of 1/a.  Every float within one ulp of 1/a, scaled by 2^19
    (exact), truncates to the same integer as the integer quotient: the
    quotient's fraction is at least 1/a, far above the scaled error."""
    for a in range(513, 1024, 2):
        r = np.float32(1.0) / np.float32(a)           # correctly rounded 1/a
        for rr in (np.nextafter(r, np.float32(0)), r, np.nextafter(r, np.float32(1))):
            assert int(np.float32(524288.0) * rr) == 524288 // a, a
