"""GPU attention alone against the oracle's attention, on the same inputs.

The decoder-level tests hold hidden rows to relative L2 1e-3, a bar set by
the reference's fast-exp SiLU (a last-bit difference can double one mlp
element).  Attention has no such amplifier, so here the GPU kernels get the
oracle's exact inputs through test hooks and are held to tight bars:

  * decode (tl_attn_decode_dev: q/k head RMSNorm, M-RoPE at the rotary
    position, K/V append at the cache position, GQA attention over the
    cache; reference kernel/decoder.c:72-118, kernel/ops.c:22-56 and
    :233-289, kernel/kv_cache.c:53-64, kernel/attention.c:172-224):
    the appended V row bit-exact, the appended K row and the attention
    output within relative L2 1e-6 and 1e-5 (only summation orders differ:
    tree sums here, sequential chains in the reference), earlier cache rows
    untouched;
  * prefill (tl_attn_prefill_dev: causal flash attention over the cache,
    kernel/attention.c:252-381): relative L2 1e-5 against the oracle's
    attention_prefill, also with the longest query tiles split in two halves
    and for a chunk attending to cached rows before it (CHUNKED_PREFILL_MODE,
    compared with the matching rows of one causal pass over all tokens).

A wrong rotation sign, a dropped norm weight, an off-by-one mask or a
misplaced softmax rescale moves these outputs by O(1), far above the bars.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
F = np.float32
NQ, NKV, HD = 16, 8, 128


def say(msg):
    print(f"[case] {msg}", flush=True)


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _decode_reference(orc, qkv, qn, kn, cos, sin, kc, vc, pos, rope_pos):
    q = orc.rmsnorm(qkv[:NQ * HD].reshape(NQ, HD), qn).reshape(-1)
    k = orc.rmsnorm(qkv[NQ * HD:(NQ + NKV) * HD].reshape(NKV, HD), kn).reshape(-1)
    v = qkv[(NQ + NKV) * HD:]
    q, k = orc.mrope_apply(q, k, cos, sin, rope_pos)
    kc = kc.copy()
    vc = vc.copy()
    kc[:, pos] = k.reshape(NKV, HD)
    vc[:, pos] = v.reshape(NKV, HD)
    return orc.attention_decode(q, kc, vc, pos + 1), kc, vc


@pytest.mark.parametrize("pos,rope_pos", [(0, 0), (63, 63), (64, 64), (130, 500), (1199, 1199), (1455, 1455),
                                          (1711, 1711), (2047, 2047)])
def test_attn_decode_matches_oracle(lin, orc, dev, pos, rope_pos):
    import torch
    say(f"attention decode pos={pos} rope_pos={rope_pos}")
    lib = lin.load_library()
    max_seq = 2048
    rng = np.random.default_rng(pos * 7 + rope_pos)
    qkv = (rng.standard_normal((NQ + 2 * NKV) * HD) * 1.5).astype(F)
    qn = (1 + 0.1 * rng.standard_normal(HD)).astype(F)
    kn = (1 + 0.1 * rng.standard_normal(HD)).astype(F)
    cos, sin = orc.rope_tables(max_seq)
    kc = np.zeros((NKV, max_seq, HD), F)
    vc = np.zeros((NKV, max_seq, HD), F)
    # earlier rows: normalised-size keys (as the norm leaves them), values O(1)
    kc[:, :pos] = rng.standard_normal((NKV, pos, HD)).astype(F)
    vc[:, :pos] = rng.standard_normal((NKV, pos, HD)).astype(F)
    want, kw, vw = _decode_reference(orc, qkv, qn, kn, cos, sin, kc, vc, pos, rope_pos)

    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    args = [t(qkv), t(qn), t(kn), t(cos), t(sin)]
    for chunk in (32, 64, 128):              # positions per work-group, every kernel variant
        assert lib.tl_attn_set_chunk(chunk) == 0
        try:
            kd, vd = t(kc), t(vc)
            out = torch.full((NQ * HD,), np.nan, dtype=torch.float32, device=dev)
            rc = lib.tl_attn_decode_dev(*[a.data_ptr() for a in args], kd.data_ptr(), vd.data_ptr(), max_seq,
                                        pos, rope_pos, out.data_ptr(), None)
            assert rc == 0, lin.check(lib, "tl_attn_decode_dev")
        finally:
            lib.tl_attn_set_chunk(0)
        _check_decode(kd.cpu().numpy(), vd.cpu().numpy(), out.cpu().numpy(), kc, vc, kw, vw, want, pos)


def _check_decode(kg, vg, og, kc, vc, kw, vw, want, pos):
    np.testing.assert_array_equal(vg[:, pos], vw[:, pos])              # V appended as is
    assert rel_l2(kg[:, pos], kw[:, pos]) <= 1e-6, rel_l2(kg[:, pos], kw[:, pos])
    np.testing.assert_array_equal(kg[:, :pos], kc[:, :pos])            # earlier rows untouched
    np.testing.assert_array_equal(vg[:, :pos], vc[:, :pos])
    assert np.all(kg[:, pos + 1:] == 0) and np.all(vg[:, pos + 1:] == 0)
    assert np.all(np.isfinite(og))
    assert rel_l2(og, want) <= 1e-5, rel_l2(og, want)
    # per head too: a head-local mistake must not hide in the global norm
    for h in range(NQ):
        assert rel_l2(og[h * HD:(h + 1) * HD], want[h * HD:(h + 1) * HD]) <= 1e-5, h


def _prefill_inputs(rng, T):
    q = (rng.standard_normal((T, NQ * HD)) * 1.2).astype(F)
    k = (rng.standard_normal((T, NKV * HD)) * 1.2).astype(F)
    v = rng.standard_normal((T, NKV * HD)).astype(F)
    return q, k, v


def _run_prefill(lin, dev, q_rows, k, v, max_seq, key0, qoff, split):
    """q_rows: the S queries; k/v: token-major rows stored at cache rows 0..T-1."""
    import torch
    lib = lin.load_library()
    S, T = q_rows.shape[0], k.shape[0]
    qkv = np.zeros((S, (NQ + 2 * NKV) * HD), F)
    qkv[:, :NQ * HD] = q_rows
    kc = np.zeros((NKV, max_seq, HD), F)
    vc = np.zeros((NKV, max_seq, HD), F)
    kc[:, :T] = k.reshape(T, NKV, HD).transpose(1, 0, 2)
    vc[:, :T] = v.reshape(T, NKV, HD).transpose(1, 0, 2)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    qd, kd, vd = t(qkv), t(kc), t(vc)
    out = torch.full((S, NQ * HD), np.nan, dtype=torch.float32, device=dev)
    rc = lib.tl_attn_prefill_dev(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), out.data_ptr(), S, max_seq, key0,
                                 qoff, 1 if split else 0, None)
    assert rc == 0, lin.check(lib, "tl_attn_prefill_dev")
    return out.cpu().numpy()


@pytest.mark.parametrize("S", [1, 64, 65, 130, 330, 1200])
@pytest.mark.parametrize("split", [False, True])
def test_attn_prefill_matches_oracle(lin, orc, dev, S, split):
    say(f"attention prefill S={S} split={split}")
    rng = np.random.default_rng(S * 3 + split)
    q, k, v = _prefill_inputs(rng, S)
    want = orc.attention_prefill(q, k, v)
    got = _run_prefill(lin, dev, q, k, v, 2048, 0, 0, split)
    assert np.all(np.isfinite(got))
    assert rel_l2(got, want) <= 1e-5, rel_l2(got, want)
    for t0 in sorted({0, S // 2, S - 1}):      # single rows: early, middle, last (longest key range)
        assert rel_l2(got[t0], want[t0]) <= 1e-5, t0


@pytest.mark.parametrize("base,S", [(64, 64), (100, 36), (1000, 200), (1136, 64)])
def test_attn_chunked_prefill_matches_oracle(lin, orc, dev, base, S):
    """A chunk of S queries at rows base.. attending to every cached row
    before it: the rows base..base+S-1 of one causal pass over base + S
    tokens."""
    say(f"attention chunked prefill base={base} S={S}")
    rng = np.random.default_rng(base + S)
    T = base + S
    q, k, v = _prefill_inputs(rng, T)
    want = orc.attention_prefill(q, k, v)[base:]
    for split in (False, True):
        got = _run_prefill(lin, dev, q[base:], k, v, 2048, 0, base, split)
        assert rel_l2(got, want) <= 1e-5, (split, rel_l2(got, want))
