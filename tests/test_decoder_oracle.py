"""CPU checks that pin the oracle's restatement of the reference's decoder
layer step (oracle/decoder_ref.c: kernel/decoder.c:33-157, kernel/ops.c,
kernel/attention.c decode path).

What pins what (no Arm machine is available to run the reference):
  * FRECPE / FRSQRTE: the architecture's accuracy bound (8-bit estimates,
    relative error < 2^-8), exact values at powers of two (the largest
    estimate, 511/512 of the reciprocal), monotonicity; the reference's Newton
    steps then reach 2^-15 (one reciprocal step) and 2^-21 (two rsqrt steps);
  * the fast exp: its closed form 2^(trunc(fma(x, log2 e, 126.94269504)) - 127)
    (Schraudolph, exponent bits only), and that it stays between 2^-1.06 and
    2^-0.06 of exp;
  * rmsnorm / mrope / attention: float64 numpy statements of the formulas;
  * the layer: the same operators composed here in Python, in the order of
    kernel/decoder.c:33-157 (the C layer must equal it bit for bit).
"""
import numpy as np
import pytest

F = np.float32


@pytest.fixture(scope="module")
def o(orc):
    return orc


def _sweep():
    rng = np.random.default_rng(0)
    return np.concatenate([2.0 ** np.arange(-100, 100, 0.173), rng.uniform(1.0, 4.0, 4000)]).astype(F)


def test_estimates_accuracy_and_powers_of_two(o):
    xs = _sweep()
    re = np.array([o.frecpe(float(x)) for x in xs], np.float64)
    rs = np.array([o.frsqrte(float(x)) for x in xs], np.float64)
    x64 = xs.astype(np.float64)
    assert np.max(np.abs(re * x64 - 1)) < 2.0 ** -8
    assert np.max(np.abs(rs * np.sqrt(x64) - 1)) < 2.0 ** -8
    for k in range(-60, 60):
        assert o.frecpe(2.0 ** k) == 2.0 ** -k * (511 / 512)
        assert o.frsqrte(4.0 ** k) == 2.0 ** -k * (511 / 512)
    # non-increasing in x over [1, 4)
    order = np.argsort(xs)
    xo = xs[order]
    m = (xo >= 1.0) & (xo < 4.0)
    assert np.all(np.diff(re[order][m]) <= 0) and np.all(np.diff(rs[order][m]) <= 0)


def test_newton_steps_of_the_reference(o):
    for x in _sweep()[::7]:
        x = float(x)
        r0 = o.frecpe(x)
        r1 = np.float32(np.float32(r0) * np.float32(o.frecps(x, r0)))
        assert abs(float(r1) * x - 1) < 2.0 ** -15
        r = o.frsqrte(x)
        for _ in range(2):
            r = float(np.float32(np.float32(r) * np.float32(o.frsqrts(float(np.float32(x * r)), r))))
        assert abs(r * np.sqrt(x) - 1) < 2.0 ** -21


def test_fast_exp_closed_form(o):
    xs = np.linspace(-100, 100, 20011).astype(F)
    for x in xs:
        xc = min(max(float(x), -88.0), 88.0)
        t = np.float32(np.float64(np.float32(xc)) * np.float64(F(1.4426950408889634)) + np.float64(F(126.94269504)))
        want = 2.0 ** (int(np.trunc(t)) - 127) if int(np.trunc(t)) > 0 else 0.0
        got = o.fast_exp(float(x))
        assert got == np.float32(want), (x, got, want)
        if -80 < x < 80:
            # floor(y - 0.0573) with y = x log2(e): 2^-1.0573 < fast/exp <= 2^-0.0573
            assert 0.4805 < got / np.exp(float(x)) <= 0.9612


def test_silu_fast_is_g_over_one_plus_fast_exp(o):
    for g in np.linspace(-30, 30, 6001).astype(F):
        g = float(g)
        want = g / (1.0 + o.fast_exp(-g))
        got = o.silu_fast(g)
        assert abs(got - want) <= 2.0 ** -14 * abs(want) + 1e-30


def test_rmsnorm_against_float64(o):
    rng = np.random.default_rng(1)
    for dim in (128, 2048):
        x = (rng.standard_normal((5, dim)) * rng.uniform(0.1, 30)).astype(F)
        w = (1 + 0.1 * rng.standard_normal(dim)).astype(F)
        got = o.rmsnorm(x, w)
        x64 = x.astype(np.float64)
        want = x64 / np.sqrt(np.mean(x64 * x64, axis=-1, keepdims=True) + 1e-6) * w
        assert np.max(np.abs(got - want) / (np.abs(want) + 1e-30)) < 2e-6


def test_rope_tables_and_apply(o):
    c, s = o.rope_tables(64)
    half = 64
    j = np.arange(half)
    inv = 1.0 / np.power(5e6, 2 * j / 128.0)
    for pos in (0, 1, 17, 63):
        # float32 inverse frequency and angle: |angle error| <= ~3 ulp of the angle
        ang = pos * inv
        tol = 3 * 2.0 ** -24 * np.maximum(ang, 1e-30) + 1.2e-7
        assert np.all(np.abs(c[pos] - np.cos(ang)) <= tol)
        assert np.all(np.abs(s[pos] - np.sin(ang)) <= tol)
    rng = np.random.default_rng(2)
    q = rng.standard_normal(16 * 128).astype(F)
    k = rng.standard_normal(8 * 128).astype(F)
    qr, kr = o.mrope_apply(q, k, c, s, 37)
    for src, got in ((q, qr), (k, kr)):
        h = src.reshape(-1, 128).astype(np.float64)
        lo, hi = h[:, :64], h[:, 64:]
        cc, ss = c[37].astype(np.float64), s[37].astype(np.float64)
        want = np.concatenate([lo * cc - hi * ss, hi * cc + lo * ss], axis=1).reshape(-1)
        assert np.max(np.abs(got - want)) < 1e-6


def test_attention_decode_against_float64(o):
    rng = np.random.default_rng(3)
    max_seq, S = 300, 257
    q = rng.standard_normal(16 * 128).astype(F)
    kc = rng.standard_normal((8, max_seq, 128)).astype(F)
    vc = rng.standard_normal((8, max_seq, 128)).astype(F)
    got = o.attention_decode(q, kc, vc, S)
    out = np.empty(16 * 128)
    for qh in range(16):
        kvh = qh // 2
        sc = kc[kvh, :S].astype(np.float64) @ q[qh * 128:(qh + 1) * 128].astype(np.float64) * 0.08838834764831843
        p = np.exp(sc - sc.max())
        p /= p.sum()
        out[qh * 128:(qh + 1) * 128] = p @ vc[kvh, :S].astype(np.float64)
    assert np.max(np.abs(got - out)) < 2e-6


def test_decode_layer_is_the_reference_composition(o):
    """The C layer equals the operators composed in the order of
    kernel/decoder.c:33-157, bit for bit (small dimensions, two steps)."""
    rng = np.random.default_rng(4)
    H, FF, nq, nkv, max_seq = 256, 384, 2, 1, 8
    KV = nkv * 128

    def quant(n, k):
        return o.quantize_rows((rng.standard_normal((n, k)) * 0.05).astype(F))
    layer = {"q_proj": quant(H, H), "k_proj": quant(KV, H), "v_proj": quant(KV, H), "o_proj": quant(H, H),
             "gate_proj": quant(FF, H), "up_proj": quant(FF, H), "down_proj": quant(H, FF),
             "input_ln": (1 + 0.1 * rng.standard_normal(H)).astype(F),
             "post_attn_ln": (1 + 0.1 * rng.standard_normal(H)).astype(F),
             "q_norm": (1 + 0.1 * rng.standard_normal(128)).astype(F),
             "k_norm": (1 + 0.1 * rng.standard_normal(128)).astype(F)}
    c, s = o.rope_tables(max_seq)
    kc = np.zeros((nkv, max_seq, 128), F)
    vc = np.zeros((nkv, max_seq, 128), F)
    kc2, vc2 = kc.copy(), vc.copy()
    h = rng.standard_normal(H).astype(F)
    h2 = h.copy()
    for step in range(2):
        h = o.decode_layer(layer, kc, vc, h, c, s, cache_len=step, rope_pos=step + 3)
        # composition
        lin = lambda x, name: o.w8a32_linear(x[None], *layer[name])[0]
        res = h2.copy()
        xn = o.rmsnorm(h2, layer["input_ln"])
        q = o.rmsnorm(lin(xn, "q_proj").reshape(-1, 128), layer["q_norm"]).reshape(-1)
        k = o.rmsnorm(lin(xn, "k_proj").reshape(-1, 128), layer["k_norm"]).reshape(-1)
        v = lin(xn, "v_proj")
        q, k = o.mrope_apply(q, k, c, s, step + 3)
        kc2[:, step] = k.reshape(nkv, 128)
        vc2[:, step] = v.reshape(nkv, 128)
        attn = o.attention_decode(q, kc2, vc2, step + 1)
        h2 = (lin(attn, "o_proj") + res).astype(F)
        res = h2.copy()
        xn = o.rmsnorm(h2, layer["post_attn_ln"])
        mlp = o.silu_mul(lin(xn, "gate_proj"), lin(xn, "up_proj"))
        h2 = (lin(mlp, "down_proj") + res).astype(F)
        np.testing.assert_array_equal(h, h2)
        np.testing.assert_array_equal(kc, kc2)
        np.testing.assert_array_equal(vc, vc2)


def test_attention_prefill_against_float64(o):
    """Causal flash attention (attention.c:252-344, 32-query x 256-key tiles,
    online softmax, polynomial exp) against a float64 softmax, across
    several key tiles and a ragged last query tile."""
    rng = np.random.default_rng(5)
    S = 300
    q = rng.standard_normal((S, 16 * 128)).astype(F)
    k = rng.standard_normal((S, 8 * 128)).astype(F)
    v = rng.standard_normal((S, 8 * 128)).astype(F)
    got = o.attention_prefill(q, k, v)
    want = np.empty((S, 16 * 128))
    for qh in range(16):
        kv = qh // 2
        Q = q[:, qh * 128:(qh + 1) * 128].astype(np.float64)
        K = k[:, kv * 128:(kv + 1) * 128].astype(np.float64)
        V = v[:, kv * 128:(kv + 1) * 128].astype(np.float64)
        sc = Q @ K.T * 0.08838834764831843
        sc[np.triu_indices(S, 1)] = -np.inf
        p = np.exp(sc - sc.max(axis=1, keepdims=True))
        want[:, qh * 128:(qh + 1) * 128] = (p / p.sum(axis=1, keepdims=True)) @ V
    assert np.max(np.abs(got - want)) < 5e-6
    # the first query attends only to itself: its output is v of position 0
    np.testing.assert_allclose(got[0].reshape(16, 128), v[0].reshape(8, 128).repeat(2, axis=0), rtol=0, atol=0)


def test_rope_tables_3d(o):
    """Per-token M-RoPE tables: dims j < 60 take the T/H/W position j % 3,
    the rest T (ops.c:128-146); sequential positions reproduce the 1-D table."""
    rng = np.random.default_rng(6)
    S = 40
    pos = np.stack([rng.integers(0, 30, S), rng.integers(0, 30, S), rng.integers(0, 30, S)]).astype(np.int32)
    c3, s3 = o.rope_tables_3d(pos)
    c1, s1 = o.rope_tables(64)
    for t in range(S):
        for j in range(64):
            sect = j % 3 if j < 60 else 0
            p = pos[sect, t]
            assert c3[t, j] == c1[p, j] and s3[t, j] == s1[p, j]
    seq = np.tile(np.arange(S, dtype=np.int32), (3, 1))
    c3, s3 = o.rope_tables_3d(seq)
    np.testing.assert_array_equal(c3, c1[:S])
    np.testing.assert_array_equal(s3, s1[:S])


def test_prefill_layer_is_the_reference_composition(o):
    """The C prefill layer equals the operators composed in the order of
    kernel/decoder.c:33-157 (PREFILL and PREFILL_3D modes), bit for bit."""
    rng = np.random.default_rng(7)
    H, FF, nkv, max_seq, S = 256, 384, 1, 48, 37
    KV = nkv * 128

    def quant(n, k):
        return o.quantize_rows((rng.standard_normal((n, k)) * 0.05).astype(F))
    layer = {"q_proj": quant(H, H), "k_proj": quant(KV, H), "v_proj": quant(KV, H), "o_proj": quant(H, H),
             "gate_proj": quant(FF, H), "up_proj": quant(FF, H), "down_proj": quant(H, FF),
             "input_ln": (1 + 0.1 * rng.standard_normal(H)).astype(F),
             "post_attn_ln": (1 + 0.1 * rng.standard_normal(H)).astype(F),
             "q_norm": (1 + 0.1 * rng.standard_normal(128)).astype(F),
             "k_norm": (1 + 0.1 * rng.standard_normal(128)).astype(F)}
    c, s = o.rope_tables(max_seq)
    pos = np.stack([np.arange(S), np.arange(S) // 4, np.arange(S) % 4]).astype(np.int32)
    tc, ts = o.rope_tables_3d(pos)
    h0 = rng.standard_normal((S, H)).astype(F)
    for mode in ("1d", "3d"):
        kc = np.zeros((nkv, max_seq, 128), F)
        vc = np.zeros_like(kc)
        if mode == "1d":
            got = o.prefill_layer(layer, kc, vc, h0, cos_tab=c, sin_tab=s, cache_len=5)
        else:
            got = o.prefill_layer(layer, kc, vc, h0, token_cos=tc, token_sin=ts, cache_len=5)
        lin = lambda x, name: o.w8a32_linear(x, *layer[name])
        res = h0.copy()
        xn = o.rmsnorm(h0, layer["input_ln"])
        q = o.rmsnorm(lin(xn, "q_proj").reshape(-1, 128), layer["q_norm"]).reshape(S, -1)
        k = o.rmsnorm(lin(xn, "k_proj").reshape(-1, 128), layer["k_norm"]).reshape(S, -1)
        v = lin(xn, "v_proj")
        for t in range(S):
            if mode == "1d":
                q[t], k[t] = o.mrope_apply(q[t], k[t], c, s, 5 + t)
            else:
                q[t], k[t] = o.mrope_apply(q[t], k[t], tc[t:t + 1], ts[t:t + 1], 0)
        np.testing.assert_array_equal(kc[:, 5:5 + S], k.reshape(S, nkv, 128).transpose(1, 0, 2))
        np.testing.assert_array_equal(vc[:, 5:5 + S], v.reshape(S, nkv, 128).transpose(1, 0, 2))
        attn = o.attention_prefill(q, k, v, nq=H // 128, nkv=nkv)
        h = (lin(attn, "o_proj") + res).astype(F)
        res = h.copy()
        xn = o.rmsnorm(h, layer["post_attn_ln"])
        mlp = o.silu_mul(lin(xn, "gate_proj").reshape(-1), lin(xn, "up_proj").reshape(-1)).reshape(S, FF)
        h = (lin(mlp, "down_proj") + res).astype(F)
        np.testing.assert_array_equal(got, h)
