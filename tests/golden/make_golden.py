"""Writes tests/golden/linear_golden.npz: small input/output vectors for the
INT8 linear path, computed by an implementation independent of oracle/.

The reference ships no tests or fixtures and cannot be compiled or run here
(AArch64 NEON + Apple Accelerate), so these vectors are derived from the
reference's source semantics with different machinery than oracle.c:
float32 arithmetic through numpy scalars (IEEE single), rounding and
accumulation with exact Python integers / fractions.

  quantizer  kernel/w8a32_kernel.c:63-108 and :139-178, kernel/w8a8_kernel.c:54-100
             scale = fl(absmax/127) (1 if absmax == 0), inv = fl(1/scale),
             k < K&~15: round-half-even(fl(x*inv)), k >= K&~15: round-half-away,
             clamped to [-127, 127]
  gemv M=1   kernel/w8a32_kernel.c:205-246: y = fl(fl(fl(acc)*ws)*xs) (+ bias, own rounding)
  w8a8 M=1   kernel/w8a8_kernel.c:181-188:  y = fma(fl(fl(acc)*ws), xs, bias)
  M>1        dequant fl(w*s) then an exact dot rounded once (the reference's
             cblas_sgemm order is unpublished; tests compare with a tolerance)

Run:  python tests/golden/make_golden.py
"""
from fractions import Fraction
import math
from pathlib import Path

import numpy as np

F = np.float32
OUT = Path(__file__).with_name("linear_golden.npz")


def f32_round(fr: Fraction) -> np.float32:
    """Nearest float32 to an exact rational, ties to even."""
    d = F(float(fr))
    cands = [np.nextafter(d, F(-np.inf)), d, np.nextafter(d, F(np.inf))]
    best = None
    for c in cands:
        err = abs(Fraction(float(c)) - fr)
        key = (err, int(np.frombuffer(F(c).tobytes(), np.uint32)[0]) & 1)
        if best is None or key < best[0]:
            best = (key, F(c))
    return best[1]


def quant_row(x: np.ndarray, clamp_main: bool = True):
    x = x.astype(F)
    K = x.size
    main_end = K & ~15
    absmax = F(0)
    for v in x:
        a = F(abs(v))
        if a > absmax:
            absmax = a
    s = F(absmax / F(127)) if absmax > 0 else F(1)
    inv = F(F(1) / s)
    q = np.zeros(K, np.int8)
    for k in range(K):
        v = float(F(x[k] * inv))          # exact float32 value, held in a double
        if k < main_end:
            r = round(v)                   # Python rounds half to even
            r = max(-128, min(127, r))
            if clamp_main:
                r = max(-127, r)
        else:
            r = int(math.copysign(math.floor(abs(v) + 0.5), v))
            r = max(-127, min(127, r))
        q[k] = r
    return q, s


def int_dot(a, b) -> int:
    return sum(int(i) * int(j) for i, j in zip(a, b))


def main():
    rng = np.random.default_rng(20240611)
    g = {}

    # --- quantizer cases -------------------------------------------------
    cases = []
    cases.append(rng.standard_normal(64).astype(F))
    cases.append(rng.standard_normal(37).astype(F))                  # tail of 5
    cases.append(rng.standard_normal(2048).astype(F))
    cases.append(np.zeros(48, F))                                     # absmax 0
    t = np.zeros(32, F); t[0] = F(127); t[1:9] = F([2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 1.5, 126.5])
    cases.append(t)                                                   # ties, s == 1
    t = np.zeros(21, F); t[0] = F(-127); t[16:21] = F([2.5, -2.5, 0.5, -0.5, 1.5])
    cases.append(t)                                                   # ties in the tail
    t = (rng.standard_normal(40) * 1e-3).astype(F); t[3] = F(-0.2)
    cases.append(t)                                                   # negative argmax
    # rows where fl(x*fl(1/s)) and fl(x/s) round to different codes
    found = []
    while len(found) < 16:
        row = rng.standard_normal(16).astype(F)
        q, s = quant_row(row)
        inv = F(F(1) / s)
        for v in row:
            a, b = float(F(v * inv)), float(F(v / s))
            if round(a) != round(b):
                found.append(row)
                break
    cases.extend(found)
    lens = np.array([c.size for c in cases], np.int64)
    g["quant_src"] = np.concatenate(cases)
    g["quant_len"] = lens
    for clamp in (1, 0):
        qs, ss = [], []
        for c in cases:
            q, s = quant_row(c, bool(clamp))
            qs.append(q); ss.append(s)
        g[f"quant_codes_c{clamp}"] = np.concatenate(qs)
        g[f"quant_scales_c{clamp}"] = np.array(ss, F)

    # --- M=1 GEMV (w8a32 batch==1) and w8a8 batch==1 ----------------------
    for tag, (N, K) in {"a": (24, 128), "b": (40, 50), "c": (16, 2048)}.items():
        x = rng.standard_normal(K).astype(F)
        w = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
        ws = rng.uniform(0.002, 0.02, N).astype(F)
        bias = rng.standard_normal(N).astype(F)
        q, xs = quant_row(x, clamp_main=False)
        acc = np.array([int_dot(w[n], q) for n in range(N)], np.int64)
        y = np.array([F(F(F(acc[n]) * ws[n]) * xs) for n in range(N)], F)
        yb = np.array([F(y[n] + bias[n]) for n in range(N)], F)
        y8 = np.array([f32_round(Fraction(float(F(F(acc[n]) * ws[n]))) * Fraction(float(xs))
                                 + Fraction(float(bias[n]))) for n in range(N)], F)
        g.update({f"gemv_{tag}_x": x, f"gemv_{tag}_w": w, f"gemv_{tag}_ws": ws,
                  f"gemv_{tag}_bias": bias, f"gemv_{tag}_codes": q, f"gemv_{tag}_xs": np.array([xs], F),
                  f"gemv_{tag}_acc": acc.astype(np.int32), f"gemv_{tag}_y": y, f"gemv_{tag}_ybias": yb,
                  f"gemv_{tag}_y8bias": y8})

    # --- M>1 (dequant then dot), exact sum rounded once -------------------
    M, N, K = 3, 20, 96
    X = rng.standard_normal((M, K)).astype(F)
    w = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    ws = rng.uniform(0.002, 0.02, N).astype(F)
    Y = np.zeros((M, N), F)
    for n in range(N):
        wd = [Fraction(float(F(F(int(w[n, k])) * ws[n]))) for k in range(K)]
        for m in range(M):
            Y[m, n] = f32_round(sum(Fraction(float(X[m, k])) * wd[k] for k in range(K)))
    g.update({"gemm_X": X, "gemm_w": w, "gemm_ws": ws, "gemm_Y": Y})

    np.savez_compressed(OUT, **g)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
