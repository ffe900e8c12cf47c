"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle.

Bars (written in each test): int8 codes and int32 accumulators bit-exact;
W8A32/W8A8 M=1 fp32 outputs bit-exact (the reference's epilogue is a fixed
sequence of IEEE roundings); M>1 fp32 outputs within relative L2 1e-5;
W8A16 fp32 outputs within 1e-5, bf16/fp16 outputs within 2e-3; lm_head argmax
identical.  Sizes are chosen so the oracle finishes in seconds; the largest
shapes are additionally checked through size-independent properties.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
F = np.float32


def say(msg):
    print(f"[case] {msg}", flush=True)


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def make(rng, M, N, K):
    x = rng.standard_normal((M, K), dtype=np.float32)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    s = rng.uniform(0.002, 0.02, N).astype(F)
    return x, w, s


def exact_epilogue(acc, ws, xs):
    """fl(fl(fl(acc) * ws[n]) * xs[m]) in float32 (numpy rounds every
    float32 product to nearest even)."""
    a = np.asarray(acc).astype(F)
    return (a * ws[None, :].astype(F)).astype(F) * xs[:, None].astype(F)


def bf16_bits(x):
    u = np.ascontiguousarray(x, F).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(b):
    return (b.astype(np.uint32) << 16).view(F)


def plant_inf(x, w, r, k_pos=9, k_neg=None):
    """Row r of x gets +Inf at column k_pos and -Inf at column k_neg (K - 5 by
    default, another K slice for K > 64), and every seventh weight row a zero
    code at k_pos: the reference's fp32 sums then give NaN (inf * 0, or
    infinite terms of both signs), +Inf and -Inf across the outputs."""
    K = x.shape[1]
    k_neg = K - 5 if k_neg is None else k_neg
    x[r, k_pos] = np.inf
    x[r, k_neg] = -np.inf
    w[::7, k_pos] = 0


def assert_nonfinite_row(got, want, tag=""):
    """A row holding Inf: NaN exactly where the oracle gives NaN, and the
    oracle's signed Inf everywhere else (all three occur)."""
    assert np.isnan(want).any() and np.isposinf(want).any() and np.isneginf(want).any(), tag
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want), err_msg=f"NaN positions {tag}")
    keep = ~np.isnan(want)
    np.testing.assert_array_equal(got[keep], want[keep], err_msg=f"signed Inf {tag}")


def test_single_hip_runtime(lin):
    """The library and torch must share one HIP runtime in the process."""
    lin.load_library()
    import torch
    assert torch.cuda.is_available()
    maps = open("/proc/self/maps").read().split("\n")
    hip = {ln.split()[-1] for ln in maps if "libamdhip64" in ln}
    assert len(hip) == 1, hip


# ---------------------------------------------------------------------------
# quantizers
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("rows,cols", [(7, 2048), (3, 6144), (5, 37), (4, 1), (2, 16), (33, 100)])
def test_quantizers_bit_exact(lin, orc, rows, cols):
    say(f"quantize rows={rows} cols={cols}")
    rng = np.random.default_rng(rows * 1000 + cols)
    w = (rng.standard_normal((rows, cols)) * rng.uniform(1e-3, 10, (rows, 1))).astype(F)
    w[0, :] = 0.0                                        # absmax 0 -> scale 1
    if cols >= 16:
        w[-1, 3] = w[-1, 3] * 0 + np.abs(w[-1]).max() * 1.0  # an exact argmax
    want_q, want_s = orc.quantize_rows(w)
    for fn in ("w8a32_quantize", "w8a8_quantize_weights", "w8a8_quantize_activations",
               "w8a16_quantize_weights"):
        q, s = lin.quantize(w, fn)
        np.testing.assert_array_equal(s, want_s, err_msg=fn)
        np.testing.assert_array_equal(q, want_q, err_msg=fn)


def test_quantizer_ties_nan_inf(lin, orc):
    say("quantize ties/nan/inf")
    rows = []
    r = np.zeros(32, F); r[0] = 127; r[1:7] = [2.5, 3.5, -2.5, -3.5, 0.5, -0.5]; rows.append(r)
    r = np.zeros(32, F); r[0] = 127; r[16:21] = [2.5, -2.5, 0.5, -0.5, 3.5]; rows.append(r)
    r = np.linspace(-3, 3, 32).astype(F); r[5] = np.nan; rows.append(r)
    r = np.ones(32, F); r[2] = np.inf; rows.append(r)
    for i, r in enumerate(rows):
        q, s = lin.quantize(r[None])
        wq, ws = orc.quantize_rows(r[None])
        np.testing.assert_array_equal(q, wq, err_msg=str(i))
        assert (s[0] == ws[0]) or (np.isinf(s[0]) and np.isinf(ws[0])), i
    # tail-only case (K=21): codes 16..20 use round-half-away
    r = np.zeros(21, F); r[0] = 127; r[16:21] = [2.5, -2.5, 0.5, -0.5, 3.5]
    q, _ = lin.quantize(r[None])
    assert list(q[0, 16:21]) == [3, -3, 1, -1, 4]


# ---------------------------------------------------------------------------
# M=1 decode GEMV (W8A32 batch==1)
# ---------------------------------------------------------------------------
DECODE_SHAPES = [(6144, 2048), (4096, 2048), (2048, 2048), (1024, 2048), (12288, 2048),
                 (2048, 6144), (37, 50), (100, 1000), (16, 64), (512, 16384), (48, 20000)]


@pytest.mark.parametrize("N,K", DECODE_SHAPES)
def test_gemv_w8a32_bit_exact(lin, orc, N, K):
    say(f"gemv w8a32 host-ABI N={N} K={K}")
    rng = np.random.default_rng(N + 7 * K)
    x, w, s = make(rng, 1, N, K)
    want, codes, xs, acc = orc.w8a32_linear(x, w, s, detail=True)
    got = lin.w8a32_linear(x, w, s)
    np.testing.assert_array_equal(got, want)
    b = rng.standard_normal(N).astype(F)
    np.testing.assert_array_equal(lin.w8a32_linear(x, w, s, bias=b), orc.w8a32_linear(x, w, s, bias=b))


@pytest.mark.parametrize("N,K", [(6144, 2048), (2048, 6144), (151936 // 16, 2048), (37, 50), (64, 16384)])
def test_gemv_accumulators_and_scale(lin, orc, dev, N, K):
    import torch
    say(f"gemv int32 acc N={N} K={K}")
    rng = np.random.default_rng(N * 3 + K)
    x, w, s = make(rng, 1, N, K)
    _, codes, xs, acc = orc.w8a32_linear(x, w, s, detail=True)
    W = lin.DeviceWeights.from_codes(w, s)
    xd = torch.from_numpy(x).to(dev)
    accd = torch.empty(N, dtype=torch.int32, device=dev)
    xsd = torch.empty(1, dtype=torch.float32, device=dev)
    lin.gemv_acc_dev(xd, W, accd, xsd)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(accd.cpu().numpy(), acc)       # exact int32
    assert xsd.cpu().numpy()[0] == xs
    W.close()


def _special_x(case, K, rng):
    x = rng.standard_normal(K).astype(F)
    if case == "ties":          # absmax 127 -> scale 1, inv 1: exact .5 ties
        x = rng.integers(-120, 120, K).astype(F) + F(0.5)
        x[7] = 127.0
    elif case == "nan":
        x[100] = np.nan
    elif case == "inf":
        x[3] = np.inf
    elif case == "denormal":    # absmax / 127 underflows: the reciprocal overflows
        x = (rng.integers(-3, 4, K) * 1e-45).astype(F)
        x[0] = F(1.4e-45)
    elif case == "zero":
        x[:] = 0.0
    elif case == "huge":
        x *= F(1e37)
    return x[None]


@pytest.mark.parametrize("case", ["ties", "nan", "inf", "denormal", "zero", "huge"])
@pytest.mark.parametrize("K", [2048, 6144, 1000])
def test_gemv_fused_quantization_special_values(lin, orc, dev, case, K):
    """The fused activation quantizer of the GEMV (the fast low-byte rounding
    and the general path it falls back to) gives the oracle's scale and
    exact accumulators on ties, NaN, Inf, underflowing and huge inputs."""
    import torch
    # denormal with K % 16: the tail's (int)lroundf(+-inf) takes the value
    # the reference's AArch64 build computes (FCVTAS to 64 bits, low 32 bits
    # kept), which the oracle restates and tests/test_oracle.py pins
    say(f"gemv fused quantization case={case} K={K}")
    rng = np.random.default_rng(K + len(case))
    N = 64
    x = _special_x(case, K, rng)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    s = rng.uniform(0.002, 0.02, N).astype(F)
    _, codes, xs, acc = orc.w8a32_linear(x, w, s, detail=True)
    W = lin.DeviceWeights.from_codes(w, s)
    accd = torch.empty(N, dtype=torch.int32, device=dev)
    xsd = torch.empty(1, dtype=torch.float32, device=dev)
    lin.gemv_acc_dev(torch.from_numpy(x).to(dev), W, accd, xsd)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(accd.cpu().numpy(), acc)
    got_xs = xsd.cpu().numpy()[0]
    assert (got_xs == xs) or (np.isnan(got_xs) and np.isnan(xs)), (got_xs, xs)
    W.close()


@pytest.mark.parametrize("rows,u", [(16, 2), (16, 4), (16, 8), (16, 12), (8, 2), (8, 4), (8, 6), (8, 8)])
@pytest.mark.parametrize("N,K", [(1000, 2048), (4100, 2040), (300, 6144), (37, 50), (129, 16384), (8, 64)])
def test_gemv_plans_bit_exact(lin, orc, rows, u, N, K):
    """Every GEMV decomposition the planner can pick (16- or 8-row work-groups,
    each batch depth, so that waves loop over batches or hold everything in
    one pair) gives the oracle's bits, for W8A32 (fused activation
    quantization) and W8A8 (given codes)."""
    say(f"gemv plan rows={rows} u={u} N={N} K={K}")
    lib = lin.load_library()
    rng = np.random.default_rng(N * 31 + K + 7 * rows + u)
    x, w, s = make(rng, 1, N, K)
    b = rng.standard_normal(N).astype(F)
    xq, xsc = orc.quantize_rows(x, clamp_main=False)
    assert lib.tl_gemv_set_plan(rows, u) == 0
    try:
        np.testing.assert_array_equal(lin.w8a32_linear(x, w, s), orc.w8a32_linear(x, w, s))
        np.testing.assert_array_equal(lin.w8a32_linear(x, w, s, bias=b), orc.w8a32_linear(x, w, s, bias=b))
        np.testing.assert_array_equal(lin.w8a8_linear(xq, xsc, w, s, bias=b),
                                      orc.w8a8_linear(xq, xsc, w, s, bias=b))
    finally:
        lib.tl_gemv_set_plan(0, 0)


def test_gemv_deterministic_and_fused_equals_concat(lin, orc, dev):
    """Run-to-run bitwise determinism (split-K counters reset), and the fused
    QKV / gate_up matrices give the concatenation of the separate GEMVs."""
    say("gemv determinism + fused==concat")
    rng = np.random.default_rng(99)
    x, wq, sq = make(rng, 1, 2048, 2048)
    _, wk, sk = make(rng, 1, 1024, 2048)
    _, wv, sv = make(rng, 1, 1024, 2048)
    y1 = lin.w8a32_linear(x, wq, sq)
    for _ in range(3):
        np.testing.assert_array_equal(lin.w8a32_linear(x, wq, sq), y1)
    wqkv = np.ascontiguousarray(np.concatenate([wq, wk, wv]))
    sqkv = np.ascontiguousarray(np.concatenate([sq, sk, sv]))
    fused = lin.w8a32_linear(x, wqkv, sqkv)
    sep = np.concatenate([y1, lin.w8a32_linear(x, wk, sk), lin.w8a32_linear(x, wv, sv)], axis=1)
    np.testing.assert_array_equal(fused, sep)


def test_lm_head_argmax(lin, orc):
    say("lm_head N=151936 K=2048")
    rng = np.random.default_rng(151936)
    x, w, s = make(rng, 1, 151936, 2048)
    want = orc.w8a32_linear(x, w, s)
    got = lin.w8a32_linear(x, w, s)
    np.testing.assert_array_equal(got, want)
    assert int(np.argmax(got)) == int(np.argmax(want))
    # 8 more hidden states: argmax identical on every row
    for i in range(8):
        xi = rng.standard_normal((1, 2048), dtype=np.float32)
        assert int(np.argmax(lin.w8a32_linear(xi, w, s))) == int(np.argmax(orc.w8a32_linear(xi, w, s)))


def test_registry_detects_in_place_update(lin, orc):
    say("registry in-place update")
    rng = np.random.default_rng(5)
    x, w, s = make(rng, 1, 256, 512)
    y0 = lin.w8a32_linear(x, w, s)
    w[:] = rng.integers(-127, 128, w.shape, dtype=np.int8)   # same pointer, new contents
    np.testing.assert_array_equal(lin.w8a32_linear(x, w, s), orc.w8a32_linear(x, w, s))
    assert not np.array_equal(y0, lin.w8a32_linear(x, w, s))


# ---------------------------------------------------------------------------
# W8A32 batch > 1 (fp32 semantics)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("M,N,K", [(2, 2048, 2048), (4, 6144, 2048), (8, 2048, 6144), (3, 100, 70),
                                   (17, 512, 2048), (64, 1024, 2048), (200, 4096, 2048),
                                   # the row-wise plane split's other widths (K = 1024 NV)
                                   (40, 300, 1024), (70, 256, 4096), (33, 130, 6144),
                                   # long K at 9..32 tokens: the planes, not the three-term split
                                   (16, 2048, 6144), (32, 2048, 6144), (24, 2048, 4096), (12, 1000, 6144),
                                   # K 4096 or > 8192 weight rows at 9..16 tokens: the planes too;
                                   # 17..64 tokens at K >= 4096: K slices on the planes GEMM
                                   (9, 2048, 4096), (12, 9000, 2048), (20, 2048, 6144), (48, 3072, 4096)])
def test_w8a32_batch_fp32(lin, orc, M, N, K):
    say(f"w8a32 batch M={M} N={N} K={K}")
    rng = np.random.default_rng(M * 13 + N + K)
    x, w, s = make(rng, M, N, K)
    want = orc.w8a32_linear(x, w, s)
    got = lin.w8a32_linear(x, w, s)
    assert rel_l2(got, want) <= 1e-5
    b = rng.standard_normal(N).astype(F)
    assert rel_l2(lin.w8a32_linear(x, w, s, bias=b), orc.w8a32_linear(x, w, s, bias=b)) <= 1e-5


@pytest.mark.parametrize("M,N,K", [(3, 32776, 200), (8, 40000, 2048), (16, 33000, 130), (48, 33000, 130),
                                   (30, 32800, 256), (64, 4100, 512), (20, 700, 2048), (16, 12288, 2048),
                                   (32, 6144, 2048), (64, 6144, 2048), (24, 12280, 2048)])
def test_small_m_wide_n(lin, orc, M, N, K):
    """M <= 64 token rows (one to four 16-row token groups per weight tile),
    also over N >= 32768 outputs (the lm_head's regime, where a work-group
    covers several 16-row weight groups) and on the mid-width weights the
    small-M kernel takes up to 12288 rows (fp32 rows at 16 tokens, int8 codes
    at 32 rows; N = 12280 ends in a partial row group): W8A32 fp32 within
    1e-5, W8A16 fp32 out within 1e-5, W8A8 within 1e-5."""
    say(f"small-M wide-N M={M} N={N} K={K}")
    rng = np.random.default_rng(M * 7 + N + K)
    x, w, s = make(rng, M, N, K)
    assert rel_l2(lin.w8a32_linear(x, w, s), orc.w8a32_linear(x, w, s)) <= 1e-5
    xb = bf16_bits(x)
    assert rel_l2(lin.w8a16_linear(xb, w, s), orc.w8a16_linear(xb, w, s)) <= 1e-5
    xq, xs = orc.quantize_rows(x)
    assert rel_l2(lin.w8a8_linear(xq, xs, w, s), orc.w8a8_linear(xq, xs, w, s)) <= 1e-5


@pytest.mark.parametrize("M,N,K", [(40, 256, 2048), (3, 32800, 2048), (7, 32800, 2048), (36, 300, 130)])
def test_w8a32_planes_special_rows(lin, orc, M, N, K):
    """Batches that run on the int8 MFMA over four int8 planes per fp32 token
    (more than 32 tokens, or an lm_head-wide N): rows of zeros, of 1e-36 and
    of 1e35 magnitude (power-of-two plane scales far from 1; the outputs stay
    normal floats, so the oracle's own rounding is fp32's), a row with one outlier
    1000x its rms are each within relative L2 1e-5 of the oracle's fp32
    GEMM (the planes hold x to about 2^-32 of the row's absmax, with an exact
    power-of-two scale); a row holding NaN gives NaN in every output, a row
    holding +Inf and -Inf gives the oracle's NaN / +Inf / -Inf output by
    output."""
    say(f"w8a32 planes special rows M={M} N={N} K={K}")
    rng = np.random.default_rng(M * 3 + N + K)
    x, w, s = make(rng, M, N, K)
    x[0] = 0.0
    x[1] *= F(1e-36)
    x[2 % M] *= F(1e35)
    if M > 3:
        x[3, 17] = F(1000.0) * np.sqrt(np.mean(x[3] ** 2))
    nan_row, inf_row = M - 1, M - 2
    x[nan_row, 5] = np.nan
    plant_inf(x, w, inf_row)
    b = rng.standard_normal(N).astype(F)
    got = lin.w8a32_linear(x, w, s, bias=b)
    want = orc.w8a32_linear(x, w, s, bias=b)
    for r in range(M):
        if r == nan_row:
            assert np.isnan(got[r]).all()
        elif r == inf_row:
            assert_nonfinite_row(got[r], want[r])
        elif r == 0:
            np.testing.assert_array_equal(got[r], b)
        else:
            assert rel_l2(got[r], want[r]) <= 1e-5, (r, rel_l2(got[r], want[r]))
    # and the same call twice gives the same bits
    np.testing.assert_array_equal(lin.w8a32_linear(x, w, s, bias=b), got)


@pytest.mark.parametrize("M,N,K", [(6, 300, 2048), (20, 2048, 2048)])
def test_w8a32_small_batch_special_rows(lin, orc, M, N, K):
    """Small batches on narrow weights (up to 32 tokens, N < 32768) split fp32
    X into three bf16 terms inside the small-M kernel: rows of zeros, of 1e-36
    and of 1e30 magnitude and a 1000x outlier row are within relative L2 1e-5
    of the oracle; a row holding NaN gives NaN in every output, a row holding
    +Inf and -Inf the oracle's NaN / +Inf / -Inf output by output.  (This
    path sums w * x before the row's weight scale, so activations with an rms
    above about 1e34 would overflow where the reference, which scales every
    weight first, stays finite.)"""
    say(f"w8a32 small-batch special rows M={M} N={N} K={K}")
    rng = np.random.default_rng(M * 5 + N + K)
    x, w, s = make(rng, M, N, K)
    x[0] = 0.0
    x[1] *= F(1e-36)
    x[2] *= F(1e30)
    x[3, 17] = F(1000.0) * np.sqrt(np.mean(x[3] ** 2))
    nan_row, inf_row = M - 1, M - 2
    x[nan_row, 5] = np.nan
    plant_inf(x, w, inf_row)
    b = rng.standard_normal(N).astype(F)
    got = lin.w8a32_linear(x, w, s, bias=b)
    want = orc.w8a32_linear(x, w, s, bias=b)
    for r in range(M):
        if r == nan_row:
            assert not np.isfinite(want[r]).any() and np.isnan(got[r]).all(), r
        elif r == inf_row:
            assert_nonfinite_row(got[r], want[r], r)
        elif r == 0:
            np.testing.assert_allclose(got[r], b, rtol=0, atol=0)
        else:
            assert rel_l2(got[r], want[r]) <= 1e-5, (r, rel_l2(got[r], want[r]))


@pytest.mark.parametrize("M,N,K", [(2, 2048, 2048), (4, 2048, 6144), (5, 300, 2048), (8, 4096, 2048),
                                   (7, 100, 68), (3, 20000, 2048), (8, 2048, 6144)])
def test_rows_digit_planes_k_slices(lin, orc, M, N, K):
    """w8a32_linear at 2..8 token rows as int8 digit planes (rows.hip) at
    every K-slice count: one slice (outputs stored directly) and 2..5 slices
    (partials merged by the row group's last work-group), each within
    relative L2 1e-5 of the oracle's fp32 GEMM, bias included; a row holding
    NaN gives NaN outputs and one holding +Inf and -Inf in different K slices
    the oracle's NaN / +Inf / -Inf output by output (the slices' partials
    merge under IEEE addition), leaving the other rows' bits unchanged; two
    calls in a row give the same bits (the arrival counters are back at
    zero); the earlier small-batch kernel (split -1) agrees too.  Work-groups
    of 2 and 3 weight row groups sharing one split of the activations
    (including a last work-group whose row groups run past N) give the same
    bits as one row group per work-group."""
    say(f"rows digit planes M={M} N={N} K={K}")
    lib = lin.load_library()
    rng = np.random.default_rng(M * 31 + N + K)
    x, w, s = make(rng, M, N, K)
    xn = x.copy()
    plant_inf(xn, w, 0)                              # zero codes in w before the oracle runs
    xn[M - 1, K // 3] = np.nan
    b = rng.standard_normal(N).astype(F)
    want = orc.w8a32_linear(x, w, s, bias=b)
    want_inf = orc.w8a32_linear(xn, w, s, bias=b)[0]
    try:
        assert lib.tl_w8a32_set_gemv2(0) == 0        # 2 rows too on the digit-row kernel
        by_split = {}
        for groups in (1, 2, 3, 0):
            assert lib.tl_rows_set_groups(groups) == 0
            for split in ((1, 2, 3, 5, -1, 0) if groups == 0 else (1, 3)):
                say(f"  groups {groups} split {split}")
                assert lib.tl_rows_set_split(split) == 0
                got = lin.w8a32_linear(x, w, s, bias=b)
                assert rel_l2(got, want) <= 1e-5, (groups, split, rel_l2(got, want))
                np.testing.assert_array_equal(lin.w8a32_linear(x, w, s, bias=b), got)
                if split in by_split:
                    np.testing.assert_array_equal(got, by_split[split])
                by_split.setdefault(split, got)
                gn = lin.w8a32_linear(xn, w, s, bias=b)
                assert np.isnan(gn[M - 1]).all(), (groups, split)
                assert_nonfinite_row(gn[0], want_inf, (groups, split))
                np.testing.assert_array_equal(gn[1:M - 1], got[1:M - 1])
    finally:
        lib.tl_rows_set_split(0)
        lib.tl_rows_set_groups(0)
        lib.tl_w8a32_set_gemv2(1)


@pytest.mark.parametrize("M", [2, 3, 4])
@pytest.mark.parametrize("N,K", [(4096, 2048), (2048, 2048), (12288, 2048), (2048, 6144), (1000, 1000),
                                 (37, 50), (300, 16384)])
def test_w8a32_token_rows_on_the_gemv(lin, orc, dev, M, N, K):
    """w8a32_linear at batch 2..4 on the GEMV's weight stream with four int8
    digit rows per fp32 token (switched on for every shape it takes here):
    bit-identical to the digit-row kernel at one K slice (the same exponent,
    digits, sums and epilogue), which is its path with the switch off, and
    within relative L2 1e-5 of the oracle's fp32 GEMM, bias included (rows of
    1e-36 and 1e35 magnitude too); a NaN in one row gives NaN in that row
    only, +Inf and -Inf in another the oracle's NaN / +Inf / -Inf output by
    output, an all-zero row gives the bias exactly; the device entry point
    gives the same bits."""
    import torch
    if M > 2 and K > 8192:
        pytest.skip("3 or 4 token rows run on the GEMV up to K = 8192")
    say(f"w8a32 {M} token rows on the GEMV N={N} K={K}")
    lib = lin.load_library()
    rng = np.random.default_rng(N * 7 + K + M)
    x, w, s = make(rng, M, N, K)
    xn = x.copy()
    plant_inf(xn, w, 0, k_neg=K // 2)                # zero codes in w before the oracle runs
    xn[M - 1, K // 3] = np.nan
    b = rng.standard_normal(N).astype(F)
    want = orc.w8a32_linear(x, w, s, bias=b)
    want_inf = orc.w8a32_linear(xn, w, s, bias=b)[0]
    assert lib.tl_w8a32_set_gemv2(2) == 0            # the GEMV for every shape it takes
    try:
        got = lin.w8a32_linear(x, w, s, bias=b)
        assert rel_l2(got, want) <= 1e-5, rel_l2(got, want)
        xz = x.copy()
        xz[0] = 0.0
        gn = lin.w8a32_linear(xn, w, s, bias=b)
        gz = lin.w8a32_linear(xz, w, s, bias=b)
        assert np.isnan(gn[M - 1]).all()
        assert_nonfinite_row(gn[0], want_inf)
        np.testing.assert_array_equal(gn[1:M - 1], got[1:M - 1])
        np.testing.assert_array_equal(gz[0], b)
        np.testing.assert_array_equal(gz[1:], got[1:])
        # a row of 1e-36 (a digit scale of about 2^149, past the float range,
        # taken in two exact steps) and one of 1e35
        xe = x.copy()
        xe[0] *= F(1e-36)
        xe[1] *= F(1e35)
        ge = lin.w8a32_linear(xe, w, s)
        we = orc.w8a32_linear(xe, w, s)
        for r in range(M):
            assert rel_l2(ge[r], we[r]) <= 1e-5, (r, rel_l2(ge[r], we[r]))
        W = lin.DeviceWeights.from_codes(w, s)
        y = torch.empty((M, N), dtype=torch.float32, device=dev)
        lin.w8a32_linear_dev(torch.from_numpy(x).to(dev), W, y, bias=torch.from_numpy(b).to(dev))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(y.cpu().numpy(), got)
        W.close()
        # the digit-row kernel's one-slice shapes (at most 96 k-blocks a slice
        # for 2 tokens, 64 for 3..4)
        if N < 32768 and K % 4 == 0 and -(-K // 64) <= (96 if M <= 2 else 64):
            assert lib.tl_w8a32_set_gemv2(0) == 0
            assert lib.tl_rows_set_split(1) == 0
            np.testing.assert_array_equal(lin.w8a32_linear(x, w, s, bias=b), got)
            np.testing.assert_array_equal(lin.w8a32_linear(xz, w, s, bias=b), gz)
            np.testing.assert_array_equal(lin.w8a32_linear(xe, w, s), ge)
    finally:
        lib.tl_w8a32_set_gemv2(1)
        lib.tl_rows_set_split(0)


def test_w8a32_prefill_rows_consistent(lin, orc):
    """1200-token prefill (fused QKV shape): rows are independent, so a
    subset computed alone matches the corresponding rows of the full call."""
    say("w8a32 prefill M=1200 N=4096 K=2048")
    rng = np.random.default_rng(1200)
    x, w, s = make(rng, 1200, 4096, 2048)
    full = lin.w8a32_linear(x, w, s)
    sub = np.r_[0:5, 597:603, 1195:1200]
    want = orc.w8a32_linear(np.ascontiguousarray(x[sub]), w, s)
    assert rel_l2(full[sub], want) <= 1e-5


@pytest.mark.parametrize("mode", ["w8a32", "w8a16_f32"])
@pytest.mark.parametrize("M,N,K", [(1200, 4096, 2048), (1024, 2048, 6144), (300, 1000, 1000)])
def test_prefill_gemm_tail_stages_and_determinism(lin, orc, dev, mode, M, N, K):
    """The last K blocks of the LDS-staged 16-bit GEMM are the ones a
    miscounted copy wait computes from a stage buffer before its copy lands
    (the buffer then still holds a K block NST stages earlier).  X is zero
    except in its last 256 columns, so such a read contributes zeros and
    misses the bar by orders of magnitude; eight repeated calls on the same
    device buffers must also agree bit for bit."""
    import torch
    say(f"prefill gemm tail stages {mode} M={M} N={N} K={K}")
    rng = np.random.default_rng(M + N + K)
    x, w, s = make(rng, M, N, K)
    x[:, : K - 256] = 0.0
    if mode == "w8a16_f32":
        x = bf16_to_f32(bf16_bits(x))           # exact in bf16, so the same oracle applies
    W = lin.DeviceWeights.from_codes(w, s)
    y = torch.empty((M, N), dtype=torch.float32, device=dev)
    if mode == "w8a32":
        xd = torch.from_numpy(x).to(dev)
        run = lambda: lin.w8a32_linear_dev(xd, W, y)
    else:
        xd = torch.from_numpy(x).to(dev).to(torch.bfloat16)
        run = lambda: lin.w8a16_linear_dev(xd, W, y)
    run()
    torch.cuda.synchronize()
    first = y.cpu().numpy().copy()
    rows = np.r_[0:4, M // 2: M // 2 + 4, M - 4:M]
    want = (x[rows].astype(np.float64) @ w.astype(np.float64).T) * s.astype(np.float64)
    assert rel_l2(first[rows], want) <= 1e-5
    for _ in range(7):
        run()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(y.cpu().numpy(), first)
    W.close()


# ---------------------------------------------------------------------------
# W8A8
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("N,K", [(6144, 2048), (2048, 6144), (37, 50)])
def test_w8a8_m1_bit_exact(lin, orc, N, K):
    say(f"w8a8 M=1 N={N} K={K}")
    rng = np.random.default_rng(N + K + 1)
    x, w, s = make(rng, 1, N, K)
    xq, xs = orc.quantize_rows(x)
    b = rng.standard_normal(N).astype(F)
    np.testing.assert_array_equal(lin.w8a8_linear(xq, xs, w, s), orc.w8a8_linear(xq, xs, w, s))
    np.testing.assert_array_equal(lin.w8a8_linear(xq, xs, w, s, bias=b),
                                  orc.w8a8_linear(xq, xs, w, s, bias=b))


@pytest.mark.parametrize("M,N,K", [(2, 512, 2048), (16, 6144, 2048), (100, 2048, 6144), (256, 6144, 2048),
                                   (45, 130, 300),
                                   # the row-wise per-token quantizer's other widths
                                   (40, 300, 1024), (70, 256, 4096)])
def test_w8a8_gemm(lin, orc, dev, M, N, K):
    import torch
    say(f"w8a8 gemm M={M} N={N} K={K}")
    rng = np.random.default_rng(M + 3 * N + K)
    x, w, s = make(rng, M, N, K)
    xq, xs = orc.quantize_rows(x)
    # int32 accumulators bit-exact
    W = lin.DeviceWeights.from_codes(w, s)
    acc = torch.empty((M, N), dtype=torch.int32, device=dev)
    lin.gemm_acc_dev(torch.from_numpy(xq).to(dev), W, acc)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(acc.cpu().numpy(), orc.int_acc(xq, w))
    # fp32 outputs through the reference ABI
    assert rel_l2(lin.w8a8_linear(xq, xs, w, s), orc.w8a8_linear(xq, xs, w, s)) <= 1e-5
    # prefill path: fp32 X quantized on the GPU, then the int8 GEMM
    y = torch.empty((M, N), dtype=torch.float32, device=dev)
    lin.w8a8_linear_f32_dev(torch.from_numpy(x).to(dev), W, y)
    torch.cuda.synchronize()
    assert rel_l2(y.cpu().numpy(), orc.w8a8_linear(xq, xs, w, s)) <= 1e-5
    # and bit-exact against the exact-integer epilogue fl(fl(fl(acc) * ws) * xs):
    # pins the codes the GPU quantizer wrote into the tiles
    np.testing.assert_array_equal(y.cpu().numpy(), exact_epilogue(orc.int_acc(xq, w), s, xs))
    W.close()


@pytest.mark.parametrize("M,N,K", [(80, 130, 300), (100, 2048, 6144), (300, 1000, 1000), (1024, 6144, 2048),
                                   (128, 2048, 2048)])
def test_w8a8_gemm_configs_bit_exact(lin, orc, dev, M, N, K):
    """Every int8 MFMA GEMM configuration (both LDS-staged layouts and the
    register-loaded weight variants with each prefetch depth) gives the exact
    int32 accumulators and the exact fp32 epilogue, on ragged shapes (M, N, K
    off the tile sizes, K shorter than the prefetch distance) and full size;
    so do K ranges split over 2..8 work-groups per tile (the planner's own
    split included), called twice each."""
    import torch
    rng = np.random.default_rng(M + N + K)
    x, w, s = make(rng, M, N, K)
    xq, xs = orc.quantize_rows(x)
    want = orc.int_acc(xq, w)
    want_y = exact_epilogue(want, s, xs)
    W = lin.DeviceWeights.from_codes(w, s)
    xqd, xd = torch.from_numpy(xq).to(dev), torch.from_numpy(x).to(dev)
    lib = lin.load_library()
    runs = [(cfg, 1) for cfg in range(8)]                       # every kernel unsplit
    runs += [(-1, sp) for sp in (0, 2, 3, 5, 8)] + [(cfg, 3) for cfg in (0, 1, 2)]   # K slices
    try:
        for cfg, split in runs:
            say(f"w8a8 gemm cfg={cfg} split={split} M={M} N={N} K={K}")
            assert lib.tl_gemm_i8_set_cfg(cfg) == 0
            assert lib.tl_gemm_i8_set_split(split) == 0
            for rep in range(2):                 # twice: the arrival counters are back at zero
                acc = torch.full((M, N), -7, dtype=torch.int32, device=dev)
                lin.gemm_acc_dev(xqd, W, acc)
                y = torch.empty((M, N), dtype=torch.float32, device=dev)
                lin.w8a8_linear_f32_dev(xd, W, y)
                torch.cuda.synchronize()
                np.testing.assert_array_equal(acc.cpu().numpy(), want)
                np.testing.assert_array_equal(y.cpu().numpy(), want_y)
    finally:
        lib.tl_gemm_i8_set_cfg(-1)
        lib.tl_gemm_i8_set_split(0)
    W.close()


@pytest.mark.parametrize("N,K", [(6144, 2048), (2048, 6144)])
def test_w8a8_prefill_full_size(lin, orc, dev, N, K):
    """The W8A8 prefill shapes at M=1024 (the gate/up-sized and the down
    projections), through the planner's own kernel choice: GPU activation
    codes and scales bit-exact, full int32 accumulators bit-exact, the fp32
    outputs equal to the exact-integer epilogue fl(fl(fl(acc) * ws) * xs) bit
    for bit, and sampled rows within 1e-5 of the oracle's w8a8_linear."""
    import torch
    say(f"w8a8 prefill M=1024 N={N} K={K}")
    rng = np.random.default_rng(1024 + N)
    x, w, s = make(rng, 1024, N, K)
    xq, xs = orc.quantize_rows(x)
    xd = torch.from_numpy(x).to(dev)
    codes = torch.empty((1024, K), dtype=torch.int8, device=dev)
    scales = torch.empty(1024, dtype=torch.float32, device=dev)
    lin.quantize_rows_dev(xd, codes, scales)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(codes.cpu().numpy(), xq)
    np.testing.assert_array_equal(scales.cpu().numpy(), xs)
    W = lin.DeviceWeights.from_codes(w, s)
    acc = torch.empty((1024, N), dtype=torch.int32, device=dev)
    lin.gemm_acc_dev(codes, W, acc)
    y = torch.empty((1024, N), dtype=torch.float32, device=dev)
    lin.w8a8_linear_f32_dev(xd, W, y)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(acc.cpu().numpy(), orc.int_acc(xq, w))
    sub = np.r_[0:4, 500:504, 1020:1024]
    want = orc.w8a8_linear(np.ascontiguousarray(xq[sub]), xs[sub], w, s)
    assert rel_l2(y.cpu().numpy()[sub], want) <= 1e-5
    np.testing.assert_array_equal(y.cpu().numpy(), exact_epilogue(acc.cpu().numpy(), s, xs))
    W.close()


# ---------------------------------------------------------------------------
# W8A16
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("M,N,K", [(1, 2048, 2048), (1, 37, 50), (8, 4096, 2048), (64, 2048, 2048),
                                   (256, 12288, 2048), (33, 200, 130)])
def test_w8a16_fp32_out(lin, orc, M, N, K):
    say(f"w8a16 fp32-out M={M} N={N} K={K}")
    rng = np.random.default_rng(M + N + K + 16)
    x, w, s = make(rng, M, N, K)
    xb = bf16_bits(x)
    want = orc.w8a16_linear(xb, w, s)
    assert rel_l2(lin.w8a16_linear(xb, w, s), want) <= 1e-5
    b = rng.standard_normal(N).astype(F)
    assert rel_l2(lin.w8a16_linear(xb, w, s, bias=b), orc.w8a16_linear(xb, w, s, bias=b)) <= 1e-5


@pytest.mark.parametrize("N,K", [(4096, 2048), (2048, 6144), (151936, 2048), (300, 16384), (37, 50), (70, 1000)])
def test_w8a16_batch1_gemv_digit_rows(lin, orc, dev, N, K):
    """w8a16_linear at batch 1 on the GEMV's weight stream with x as four int8
    digit rows (gemv.hip plane mode): within relative L2 1e-5 of the oracle
    (the reference's bf16 dot products) with and without bias, also with the
    bf16 / fp16 MFMA kernel switched in (tl_w8a16_set_gemv(0)) for the same
    inputs; bf16 and fp16 outputs within 2e-3; a zero row gives the bias
    exactly, a row of 1e-30 magnitude stays within 1e-5, a NaN in x gives NaN
    outputs, and +Inf and -Inf in x the oracle's NaN / +Inf / -Inf output by
    output (on both kernels)."""
    import torch
    say(f"w8a16 batch-1 GEMV N={N} K={K}")
    lib = lin.load_library()
    rng = np.random.default_rng(N + K)
    x, w, s = make(rng, 1, N, K)
    xb = bf16_bits(x)
    b = rng.standard_normal(N).astype(F)
    want = orc.w8a16_linear(xb, w, s)
    wantb = orc.w8a16_linear(xb, w, s, bias=b)
    try:
        for on in (1, 0):
            assert lib.tl_w8a16_set_gemv(on) == 0
            assert rel_l2(lin.w8a16_linear(xb, w, s), want) <= 1e-5, on
            assert rel_l2(lin.w8a16_linear(xb, w, s, bias=b), wantb) <= 1e-5, on
    finally:
        lib.tl_w8a16_set_gemv(1)
    z = np.zeros_like(xb)
    np.testing.assert_array_equal(lin.w8a16_linear(z, w, s, bias=b), b[None, :])
    tiny = bf16_bits(x * F(1e-30))
    assert rel_l2(lin.w8a16_linear(tiny, w, s), orc.w8a16_linear(tiny, w, s)) <= 1e-5
    xx = x.copy()
    xx[0, K // 2] = np.nan
    assert np.isnan(lin.w8a16_linear(bf16_bits(xx), w, s)).all()
    xx = x.copy()
    wi = w.copy()
    plant_inf(xx, wi, 0)
    want_inf = orc.w8a16_linear(bf16_bits(xx), wi, s, bias=b)[0]
    try:
        for on in (1, 0):
            assert lib.tl_w8a16_set_gemv(on) == 0
            assert_nonfinite_row(lin.w8a16_linear(bf16_bits(xx), wi, s, bias=b)[0], want_inf, on)
    finally:
        lib.tl_w8a16_set_gemv(1)
    # device path: bf16 / fp16 x with bf16 / fp16 out
    W = lin.DeviceWeights.from_codes(w, s)
    xt = torch.from_numpy(x).to(dev).to(torch.bfloat16)
    y = torch.empty((1, N), dtype=torch.bfloat16, device=dev)
    lin.w8a16_linear_dev(xt, W, y)
    torch.cuda.synchronize()
    assert rel_l2(y.float().cpu().numpy(), want) <= 2e-3
    xh = x.astype(np.float16)
    wantf = (xh.astype(np.float64) @ w.astype(np.float64).T) * s.astype(np.float64)
    yh = torch.empty((1, N), dtype=torch.float16, device=dev)
    lin.w8a16_linear_dev(torch.from_numpy(xh).to(dev), W, yh)
    yf = torch.empty((1, N), dtype=torch.float32, device=dev)
    lin.w8a16_linear_dev(torch.from_numpy(xh).to(dev), W, yf)
    torch.cuda.synchronize()
    assert rel_l2(yh.float().cpu().numpy(), wantf) <= 2e-3
    assert rel_l2(yf.cpu().numpy(), wantf) <= 1e-5
    W.close()


def row_rel_l2(got, want):
    """Relative L2 error of every row (float64)."""
    g = np.asarray(got, np.float64)
    w = np.asarray(want, np.float64)
    return np.linalg.norm(g - w, axis=1) / np.maximum(np.linalg.norm(w, axis=1), 1e-30)


@pytest.mark.parametrize("M", [1, 8, 64, 256, 1024])
@pytest.mark.parametrize("N", [2048, 4096, 12288])
def test_w8a16_bf16_fp16(lin, orc, dev, M, N):
    """Every point of the W8A16 sweep (K=2048), every output row, against a
    float64 product of the 16-bit X with the int8 codes times the row scale
    (the reference's w8a16_gemm: X widened exactly, W dequantized, SGEMM;
    w8a16_kernel.c:187-216): bf16 X with bf16 out and fp16 X with fp16 out
    within relative L2 2e-3 in every row, bf16 X with fp32 out within 1e-5 in
    every row.  At M = 1024 x N = 12288 that is every M tile of the
    column-split GEMM in its XCD-grouped launch order."""
    import torch
    K = 2048
    say(f"w8a16 bf16/fp16/fp32-out M={M} N={N} K={K}, all rows")
    rng = np.random.default_rng(M * 7 + N)
    x, w, s = make(rng, M, N, K)
    W = lin.DeviceWeights.from_codes(w, s)
    wt = np.ascontiguousarray(w.astype(np.float64).T)
    s64 = s.astype(np.float64)
    # bf16 X: bf16 out (2e-3) and fp32 out (1e-5)
    xt = torch.from_numpy(x).to(dev).to(torch.bfloat16)
    want = (xt.float().cpu().numpy().astype(np.float64) @ wt) * s64
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    y32 = torch.empty((M, N), dtype=torch.float32, device=dev)
    lin.w8a16_linear_dev(xt, W, y)
    lin.w8a16_linear_dev(xt, W, y32)
    torch.cuda.synchronize()
    e = row_rel_l2(y.float().cpu().numpy(), want)
    assert e.max() <= 2e-3, (int(e.argmax()), float(e.max()))
    e = row_rel_l2(y32.cpu().numpy(), want)
    assert e.max() <= 1e-5, (int(e.argmax()), float(e.max()))
    # fp16 X, fp16 out
    xh = x.astype(np.float16)
    wantf = (xh.astype(np.float64) @ wt) * s64
    yh = torch.empty((M, N), dtype=torch.float16, device=dev)
    lin.w8a16_linear_dev(torch.from_numpy(xh).to(dev), W, yh)
    torch.cuda.synchronize()
    e = row_rel_l2(yh.float().cpu().numpy(), wantf)
    assert e.max() <= 2e-3, (int(e.argmax()), float(e.max()))
    W.close()


@pytest.mark.parametrize("path,K", [("w8a8_codes", 1000), ("w8a32", 20000)])
def test_batch1_padded_paths_capture_into_a_graph(lin, orc, dev, path, K):
    """The batch-1 paths that pad the activation codes in the work-space
    (W8A8 on caller codes with K % 64 != 0; W8A32 with K > 16384, whose
    codes are made by a separate quantization launch) record only kernel
    nodes when captured: the graph, replayed three times with new inputs
    written by eager work between the replays, gives the eager result of
    each input bit for bit, and the oracle's."""
    import torch
    say(f"batch-1 padded path under graph capture: {path} K={K}")
    rng = np.random.default_rng(K + 7)
    N = 512
    _, w, s = make(rng, 1, N, K)
    W = lin.DeviceWeights.from_codes(w, s)
    st = torch.cuda.Stream()
    y = torch.empty((1, N), dtype=torch.float32, device=dev)
    if path == "w8a8_codes":
        xq = torch.empty((1, K), dtype=torch.int8, device=dev)
        xs = torch.empty(1, dtype=torch.float32, device=dev)

        def call():
            lin.w8a8_linear_dev(xq, xs, W, y, stream=st)

        def put(x):
            q, sc = orc.quantize_rows(x)
            xq.copy_(torch.from_numpy(q))
            xs.copy_(torch.from_numpy(sc))
            return orc.w8a8_linear(q, sc, w, s)
    else:
        xd = torch.empty((1, K), dtype=torch.float32, device=dev)

        def call():
            lin.w8a32_linear_dev(xd, W, y, stream=st)

        def put(x):
            xd.copy_(torch.from_numpy(x))
            return orc.w8a32_linear(x, w, s)
    xs0 = rng.standard_normal((1, K), dtype=np.float32)
    put(xs0)
    torch.cuda.synchronize()
    with torch.cuda.stream(st):
        call()                                   # the work-space exists before the capture
    st.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        call()
    torch.cuda.synchronize()
    for r in range(3):
        x = (rng.standard_normal((1, K)) * (0.5 + r)).astype(np.float32)
        want = put(x)
        torch.cuda.synchronize()
        with torch.cuda.stream(st):
            call()
        st.synchronize()
        eager = y.cpu().numpy().copy()
        y.fill_(np.nan)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(y.cpu().numpy(), eager)
        np.testing.assert_array_equal(eager, want)
    del g
    W.close()


@pytest.mark.parametrize("M,N,K", [(64, 2048, 2048), (200, 1000, 1000), (200, 1000, 2048), (256, 4096, 2048)])
def test_w8a16_k_slices(lin, orc, dev, M, N, K):
    """The 16-bit GEMM with its K range split over 1..4 work-groups per tile
    (every tile configuration, forced through tl_gemm_b16_set_plan: the
    LDS-staged kernel's 0..2 and the column-split kernel's 4..8, which K not a
    multiple of 64 runs on configuration 0's kernel; uneven slices where the
    K blocks do not divide): fp32 out within 1e-5 and bf16
    out within 2e-3 of a float64 product in every row, and a repeated call
    bit-identical (the last work-group to arrive adds the slices in slice
    order, whichever it is)."""
    import torch
    lib = lin.load_library()
    rng = np.random.default_rng(M * 3 + N + K)
    x, w, s = make(rng, M, N, K)
    W = lin.DeviceWeights.from_codes(w, s)
    xt = torch.from_numpy(x).to(dev).to(torch.bfloat16)
    want = (xt.float().cpu().numpy().astype(np.float64) @ w.astype(np.float64).T) * s.astype(np.float64)
    y32 = torch.empty((M, N), dtype=torch.float32, device=dev)
    yb = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    try:
        for cfg in (0, 1, 2, 4, 5, 6, 7, 8):
            for split in (1, 2, 3, 4):
                say(f"w8a16 K slices M={M} N={N} K={K} cfg={cfg} split={split}")
                assert lib.tl_gemm_b16_set_plan(cfg, split) == 0
                lin.w8a16_linear_dev(xt, W, y32)
                lin.w8a16_linear_dev(xt, W, yb)
                torch.cuda.synchronize()
                first = y32.cpu().numpy().copy()
                e = row_rel_l2(first, want)
                assert e.max() <= 1e-5, (cfg, split, int(e.argmax()), float(e.max()))
                e = row_rel_l2(yb.float().cpu().numpy(), want)
                assert e.max() <= 2e-3, (cfg, split, int(e.argmax()), float(e.max()))
                y32.fill_(np.nan)
                lin.w8a16_linear_dev(xt, W, y32)
                torch.cuda.synchronize()
                np.testing.assert_array_equal(y32.cpu().numpy(), first)
    finally:
        lib.tl_gemm_b16_set_plan(-1, 0)
    W.close()


SMALL_B16_SHAPES = [100 * r + 10 * t + u for r in (1, 2, 4) for t in (1, 2, 4) for u in (2, 4)
                    if u == 2 or t == 1 or r * t <= 8]


def test_w8a16_rows_past_32bit_offsets(lin, orc, dev):
    """X of more than 4 GiB (2^20 + 40 rows of 2048 bf16): the tiled kernels'
    copies address X with 32-bit per-lane offsets from a per-stage base, so
    such X takes the general path with 64-bit addresses.  The first and the
    last rows (past 2^32 bytes) within 1e-5 of a float64 product."""
    import torch
    M, N, K = (1 << 20) + 40, 48, 2048
    say(f"w8a16 rows past 32-bit offsets M={M} N={N} K={K}")
    rng = np.random.default_rng(77)
    _, w, s = make(rng, 1, N, K)
    W = lin.DeviceWeights.from_codes(w, s)
    xt = torch.randn((M, K), device=dev, dtype=torch.float32, generator=torch.Generator(device=dev).manual_seed(5)
                     ).to(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.float32, device=dev)
    lin.w8a16_linear_dev(xt, W, y)
    torch.cuda.synchronize()
    for sl in (slice(0, 40), slice(M - 40, M)):
        xs = xt[sl].float().cpu().numpy().astype(np.float64)
        want = (xs @ w.astype(np.float64).T) * s.astype(np.float64)
        e = row_rel_l2(y[sl].cpu().numpy(), want)
        assert e.max() <= 1e-5, (sl, int(e.argmax()), float(e.max()))
    del xt, y
    torch.cuda.empty_cache()
    W.close()


@pytest.mark.parametrize("M,N,K", [(96, 2048, 2048), (128, 1000, 1000), (200, 2000, 2112), (40, 4096, 2048),
                                   (17, 300, 192)])
def test_w8a16_small_kernel_shapes(lin, orc, dev, M, N, K):
    """W8A16 batches of 17..256 tokens on the streamed small-M kernel (token
    rows spread over the grid's y extent): the planner's choice and every
    forced work-group shape (tl_gemm_b16_set_plan(3, 100 R + 10 TG + U)),
    ragged M, N and K included: fp32 out within 1e-5 and bf16 out within 2e-3
    of a float64 product in every row, with and without bias; fp16 X with fp16
    out within 2e-3; a repeated call bit-identical."""
    import torch
    lib = lin.load_library()
    rng = np.random.default_rng(M * 5 + N + K)
    x, w, s = make(rng, M, N, K)
    b = rng.standard_normal(N).astype(F)
    W = lin.DeviceWeights.from_codes(w, s)
    xt = torch.from_numpy(x).to(dev).to(torch.bfloat16)
    bd = torch.from_numpy(b).to(dev)
    want = (xt.float().cpu().numpy().astype(np.float64) @ w.astype(np.float64).T) * s.astype(np.float64)
    wantb = want + b.astype(np.float64)
    xh = torch.from_numpy(x.astype(np.float16)).to(dev)
    wanth = (x.astype(np.float16).astype(np.float64) @ w.astype(np.float64).T) * s.astype(np.float64)
    y32 = torch.empty((M, N), dtype=torch.float32, device=dev)
    yb = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    yh = torch.empty((M, N), dtype=torch.float16, device=dev)
    try:
        for cfg, code in [(-1, 0), (3, 0)] + [(3, c) for c in SMALL_B16_SHAPES]:
            say(f"w8a16 small kernel M={M} N={N} K={K} cfg={cfg} shape={code}")
            assert lib.tl_gemm_b16_set_plan(cfg, code) == 0
            lin.w8a16_linear_dev(xt, W, y32)
            lin.w8a16_linear_dev(xt, W, yb)
            lin.w8a16_linear_dev(xh, W, yh)
            torch.cuda.synchronize()
            first = y32.cpu().numpy().copy()
            e = row_rel_l2(first, want)
            assert e.max() <= 1e-5, (code, int(e.argmax()), float(e.max()))
            e = row_rel_l2(yb.float().cpu().numpy(), want)
            assert e.max() <= 2e-3, (code, int(e.argmax()), float(e.max()))
            e = row_rel_l2(yh.float().cpu().numpy(), wanth)
            assert e.max() <= 2e-3, (code, int(e.argmax()), float(e.max()))
            lin.w8a16_linear_dev(xt, W, y32, bias=bd)
            torch.cuda.synchronize()
            e = row_rel_l2(y32.cpu().numpy(), wantb)
            assert e.max() <= 1e-5, (code, int(e.argmax()), float(e.max()))
            y32.fill_(np.nan)
            lin.w8a16_linear_dev(xt, W, y32)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(y32.cpu().numpy(), first)
    finally:
        lib.tl_gemm_b16_set_plan(-1, 0)
    W.close()


@pytest.mark.parametrize("M,N,K", [(1024, 6144, 2048), (1024, 2048, 6144), (300, 1000, 1000)])
def test_w8a8_quantize_tiles_then_gemm(lin, orc, dev, M, N, K):
    """The two halves of tl_w8a8_linear_f32_dev (per-token codes into the
    activation tile layout, then the GEMM on them) give its outputs bit for
    bit, bias included; the token scales are the oracle's
    w8a8_quantize_activations scales."""
    import torch
    say(f"w8a8 quantize tiles + GEMM M={M} N={N} K={K}")
    lib = lin.load_library()
    rng = np.random.default_rng(M + N + K + 88)
    x, w, s = make(rng, M, N, K)
    b = rng.standard_normal(N).astype(F)
    W = lin.DeviceWeights.from_codes(w, s)
    xd = torch.from_numpy(x).to(dev)
    bd = torch.from_numpy(b).to(dev)
    tiles = torch.empty(lib.tl_w8a8_tiles_bytes(M, K), dtype=torch.uint8, device=dev)
    scales = torch.empty(-(-M // 16) * 16, dtype=torch.float32, device=dev)
    y_full = torch.empty((M, N), dtype=torch.float32, device=dev)
    y_split = torch.empty((M, N), dtype=torch.float32, device=dev)
    lin.w8a8_linear_f32_dev(xd, W, y_full, bias=bd)
    lin.w8a8_quantize_tiles_dev(xd, tiles, scales)
    lin.w8a8_linear_tiles_dev(tiles, scales, W, y_split, bias=bd)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y_split.cpu().numpy(), y_full.cpu().numpy())
    _, xs = orc.quantize_rows(x)
    np.testing.assert_array_equal(scales.cpu().numpy()[:M], xs)
    W.close()
