"""Benchmark of the INT8 linear path on one MI355X.

Workload (the metric's configuration; a "step" = W8A32 batch==1 GEMVs):
  the decode projection set of one Qwen3-VL-2B text layer plus the lm_head,
  QKV 4096x2048, O 2048x2048, gate_up 12288x2048, down 2048x6144, lm_head
  151936x2048 (361.5 MB of int8 weights and scales), per-row fp32 scales,
  fp32 activations ~N(0,1) resident in HBM, synthetic data.  Step i (5 GEMV
  launches) runs layer copy i % 28 of 28 distinct ones plus lm_head copy
  i % 2 of two, so every step's weights come from HBM (1.72 GB of layers and
  622 MB of lm_heads, far beyond the 256 MB Infinity Cache).  The timed steps
  are captured back to back in one HIP graph, as the decoder captures its
  layers; the graph is replayed 5 times, each replay timed on its own, and the
  median is the figure.  The same steps replayed as one graph each (a graph
  launch per 5 kernels) are reported as `graph_per_step`.
Also the full decoder's step, 28 layers + lm_head (113 launches, one graph):
  `decode_step_28_layers`.

value   = algorithmic bytes of one step / step time (GB/s); bytes per GEMV
          launch are N*K + 4N + 4K + 4N (weights, scales, x, y).
roofline: the GEMV kernel family (every launch is a GEMV), average bytes per
          launch over its average launch duration, against the 8 TB/s HBM
          peak.  The duration comes from the committed rocprofv3 kernel trace
          of this command (profiles/gemv_timed_steps_kernel_trace.md, written
          by --summarize-trace: the GEMV durations between the marker launches
          that bracket each timed replay) while it was taken on the current
          GEMV sources; `roofline.live` holds the same ratio on this run's
          HIP-event step time (launch gaps included).
Also: W8A8 prefill TOPS (M=1024; N=6144,K=2048 and N=2048,K=6144; includes
the per-token quantization kernel), and the CPU baseline (the oracle's M=1
GEMV, OpenMP on the host cores) on a bounded sample.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
BF16_PEAK_TFLOPS = 2500.0
COPY_PROBE_BYTES = 512 << 20
TRAFFIC_SUMMARY = ROOT / "profiles" / "gemv_decode_step_traffic.md"


# the GEMV kernel's sources: the traffic figure holds for the build it was measured on
GEMV_SOURCES = [ROOT / "typhoon-ocr-server_amd" / "csrc" / "gemv.hip", ROOT / "typhoon-ocr-server_amd" / "csrc" / "tl_common.h"]


def gemv_sources_sha256():
    h = hashlib.sha256()
    for p in GEMV_SOURCES:
        h.update(p.read_bytes())
    return h.hexdigest()


def measured_traffic():
    """HBM bytes per GEMV launch measured with rocprofv3 --pmc FETCH_SIZE and
    WRITE_SIZE on `bench.py --traffic-probe` (counters scaled by what they
    read for a 512 MiB copy), recorded in the profile summary together with
    the SHA-256 of the GEMV sources it was measured on.  Returns (bytes, note):
    bytes is None when the summary is absent or the sources changed since."""
    rec = {}
    try:
        for line in TRAFFIC_SUMMARY.read_text().splitlines():
            if ":" in line and line.split(":", 1)[0] in ("traffic_bytes_per_launch", "gemv_sources_sha256"):
                k, v = line.split(":", 1)
                rec[k] = v.strip()
    except OSError:
        return None, "no traffic summary"
    if "traffic_bytes_per_launch" not in rec:
        return None, "no traffic figure in the summary"
    if rec.get("gemv_sources_sha256") != gemv_sources_sha256():
        return None, "stale: the GEMV sources changed since the counters were taken"
    return float(rec["traffic_bytes_per_launch"]), "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, same GEMV sources"


# The timed steps' kernel trace: `bench.py --summarize-trace` writes this
# summary from a rocprofv3 --kernel-trace run of the benchmark's own command.
TRACE_SUMMARY = ROOT / "profiles" / "gemv_timed_steps_kernel_trace.md"
TIMED_REPLAYS = 5
MARKER_BYTES = 4096        # the trace marker: one 256-thread work-group reading 4 KiB


class TraceMarker:
    """A launch that brackets each timed replay in a kernel trace: the plain
    streaming read kernel on one work-group (every other launch of it in
    this benchmark uses 256 or more), outside the HIP events."""

    def __init__(self, lin, torch, dev):
        self.lib = lin.load_library()
        self.lin = lin
        self.buf = torch.ones(MARKER_BYTES, dtype=torch.uint8, device=dev)
        self.sink = torch.zeros(1, dtype=torch.int32, device=dev)

    def launch(self, stream):
        rc = self.lib.tl_stream_read_dev(self.buf.data_ptr(), MARKER_BYTES, 1, 4, self.sink.data_ptr(),
                                         stream.cuda_stream)
        assert rc == 0, self.lin.check(self.lib, "tl_stream_read_dev")


def read_summary_fields(path, keys):
    rec = {}
    for line in path.read_text().splitlines():
        if ":" in line and line.split(":", 1)[0] in keys:
            k, v = line.split(":", 1)
            rec[k] = v.strip()
    return rec


def profiled_step_kernel_us(steps):
    """GEMV kernel time of one benchmark step (us) from the committed kernel
    trace summary, or None with the reason: absent, taken on other GEMV
    sources, or at another step count."""
    try:
        rec = read_summary_fields(TRACE_SUMMARY, ("kernel_us_per_step", "gemv_sources_sha256", "steps",
                                                  "timed_replays", "lm_head_copies"))
    except OSError:
        return None, "no kernel trace summary"
    if "kernel_us_per_step" not in rec:
        return None, "no kernel_us_per_step in the trace summary"
    if rec.get("gemv_sources_sha256") != gemv_sources_sha256():
        return None, "trace summary stale: the GEMV sources changed since it was taken"
    if rec.get("steps") != str(steps) or rec.get("lm_head_copies") != str(LM_COPIES):
        return None, f"trace summary taken at steps={rec.get('steps')}, not {steps}"
    return float(rec["kernel_us_per_step"]), (f"median over its {rec.get('timed_replays')} timed replays of "
                                              f"the summed GEMV durations per step")


def summarize_trace(csv_path, steps, cmd):
    """Markdown summary of the timed replays in a rocprofv3 kernel trace of
    this benchmark: the launches between each pair of marker launches, per
    shape (told apart by grid size) and per step."""
    import csv
    rows = list(csv.DictReader(open(csv_path)))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    n_per = len(LAYER_SHAPES) + 1
    marks = [i for i, r in enumerate(rows)
             if "stream_read_kernel" in r["Kernel_Name"] and int(r["Grid_Size_X"]) == 256]
    if len(marks) < 2 or len(marks) % 2:
        raise SystemExit(f"{len(marks)} marker launches in the trace; expected pairs")
    grid_shape = {}
    for (name, N, K) in LAYER_SHAPES + [LM_HEAD]:
        grid_shape.setdefault(name, N)
    reps, per = [], {}
    for a, b in zip(marks[0::2], marks[1::2]):
        seg = [r for r in rows[a + 1:b] if "gemv_i8_kernel" in r["Kernel_Name"]]
        if len(seg) != steps * n_per or len(seg) != b - a - 1:
            raise SystemExit(f"timed replay holds {b - a - 1} launches ({len(seg)} GEMV); expected {steps * n_per}")
        durs = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3 for r in seg]
        span = (int(seg[-1]["End_Timestamp"]) - int(seg[0]["Start_Timestamp"])) * 1e-3
        reps.append((sum(durs) / steps, span / steps))
        for j, (r, d) in enumerate(zip(seg, durs)):
            shape = (LAYER_SHAPES + [LM_HEAD])[j % n_per]
            per.setdefault(shape, {"kernel": r["Kernel_Name"], "grid": int(r["Grid_Size_X"]), "d": []})["d"].append(d)
    k_step = float(np.median([k for k, _ in reps]))
    s_step = float(np.median([s for _, s in reps]))
    step_bytes = sum(gemv_bytes(N, K) for (_, N, K) in LAYER_SHAPES + [LM_HEAD])
    out = ["# GEMV timed steps: kernel durations (rocprofv3 --kernel-trace)", "",
           "Command (MI355X, one GPU):", "", "```", cmd, "```", "",
           f"Workload: the benchmark's timed steps. Step i is layer copy i % {LAYERS}'s projection set "
           "(QKV 4096x2048, O 2048x2048, gate_up 12288x2048, down 2048x6144) plus lm_head 151936x2048 "
           f"copy i % {LM_COPIES}, W8A32 batch 1, {steps} steps captured back to back in one HIP graph; "
           f"{len(reps)} timed replays, each bracketed by a one-work-group `stream_read_kernel` marker "
           "launch outside the HIP events. This summary counts the launches between each pair of "
           "markers only (every one a `gemv_i8_kernel`).", "",
           "| shape | kernel | grid threads | launches | avg us | median us | min us |",
           "|---|---|---|---|---|---|---|"]
    for (name, N, K), rec in per.items():
        d = rec["d"]
        kname = rec["kernel"].split("(")[0].replace("tl::", "")
        out.append(f"| {name} {N}x{K} | `{kname}` | {rec['grid']} | {len(d)} | {np.mean(d):.2f} | "
                   f"{np.median(d):.2f} | {np.min(d):.2f} |")
    out += ["", "Per timed replay (us per step): GEMV kernel time summed / span from the first launch's "
            "start to the last launch's end:", ""]
    out += [f"- replay {i}: {k:.2f} / {s:.2f}" for i, (k, s) in enumerate(reps)]
    out += ["", "Figures bench.py reads (median over the timed replays):", "",
            f"kernel_us_per_step: {k_step:.3f}",
            f"span_us_per_step: {s_step:.3f}",
            f"bytes_per_step: {step_bytes}",
            f"frac_hbm_from_kernel_time: {step_bytes / (k_step * 1e-6) / 1e9 / HBM_PEAK_GBS:.4f}",
            f"steps: {steps}",
            f"timed_replays: {len(reps)}",
            f"lm_head_copies: {LM_COPIES}",
            f"gemv_sources_sha256: {gemv_sources_sha256()}", ""]
    return "\n".join(out)


LAYERS = 28
LAYER_SHAPES = [("qkv", 4096, 2048), ("o", 2048, 2048), ("gate_up", 12288, 2048), ("down", 2048, 6144)]
LM_HEAD = ("lm_head", 151936, 2048)
LM_COPIES = 2
METRIC = "INT8 GEMV HBM GB/s + decode tok/s; W8A8 prefill TOPS (Qwen3-VL-2B decoder)"


def gemv_bytes(N, K):
    return N * K + 4 * N + 4 * K + 4 * N


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def build_decode_set(lin, torch, dev, seed=0):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    items = []
    # two lm_head copies: the timed steps alternate them (step i reads copy
    # i % 2), so no step finds its lm_head lines left in the Infinity Cache
    shapes = [(f"l{l}.{n}", N, K) for l in range(LAYERS) for (n, N, K) in LAYER_SHAPES] + [LM_HEAD] * LM_COPIES
    for name, N, K in shapes:
        w = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
        s = torch.rand(N, device=dev, generator=g) * 0.018 + 0.002
        W = lin.DeviceWeights.from_codes(w, s)
        del w
        x = torch.randn((1, K), device=dev, generator=g)
        y = torch.empty((1, N), device=dev)
        items.append((name, N, K, W, x, y))
    return items


def run_step(lin, items, stream):
    for (_, _, _, W, x, y) in items:
        lin.w8a32_linear_dev(x, W, y, stream=stream)


def time_shapes(lin, torch, items, dev):
    """Average launch duration per decode shape: the launches of one shape
    (its 28 distinct matrices; the lm_head alternating with a second copy of
    it, so that every launch reads HBM) captured back to back in a HIP graph
    of >= 40 launches and replayed (time_graph)."""
    by = {}
    for it in items:
        by.setdefault(it[0].split(".")[-1], []).append(it)
    out = {}
    for key, its in by.items():
        extra = []
        if len(its) == 1:
            (_, N, K, W, x, y) = its[0]
            w2 = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev)
            s2 = torch.rand(N, device=dev) * 0.018 + 0.002
            extra = [lin.DeviceWeights.from_codes(w2, s2)]
            del w2
        Ws = [it[3] for it in its] + extra
        x, y = its[0][4], its[0][5]
        t = time_graph(torch, lambda i, st: lin.w8a32_linear_dev(x, Ws[i], y, stream=st), len(Ws))
        out[key] = (its[0][1], its[0][2], t)
        for W in extra:
            W.close()
    return out


def bench_lm_head_greedy(lin, torch, W, K, dev, stream, reps=20):
    """The fused greedy step (final RMSNorm, lm_head GEMV with per-work-group
    argmax keys, key reduction: three launches) against the plain lm_head
    GEMV, each captured in a HIP graph and replayed, alternating between two
    distinct lm_head matrices (622 MB, beyond the 256 MB Infinity Cache)."""
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    w2 = torch.randint(-127, 128, (W.rows, K), dtype=torch.int8, device=dev, generator=g)
    s2 = torch.rand(W.rows, device=dev, generator=g) * 0.018 + 0.002
    W2 = lin.DeviceWeights.from_codes(w2, s2)
    del w2
    Ws = (W, W2)
    h = torch.randn(K, device=dev, generator=g)
    nw = 1.0 + 0.1 * torch.randn(K, device=dev, generator=g)
    tok = torch.empty(1, dtype=torch.int32, device=dev)
    x = torch.randn((1, K), device=dev, generator=g)
    y = torch.empty((1, W.rows), device=dev)
    out = {}
    for name, fn in (("fused_rmsnorm_gemv_argmax", lambda Wi: lin.lm_head_argmax_dev(h, nw, Wi, tok, stream=stream)),
                     ("gemv_logits_only", lambda Wi: lin.w8a32_linear_dev(x, Wi, y, stream=stream))):
        with torch.cuda.stream(stream):
            fn(W)
            fn(W2)
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(reps):
                fn(Ws[i & 1])
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(3):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        t = e0.elapsed_time(e1) * 1e-3 / (3 * reps)
        b = gemv_bytes(W.rows, K)
        out[name] = {"us": round(t * 1e6, 2), "GBps": round(b / t / 1e9, 1)}
        del graph
    W2.close()
    out["returns"] = "int32 token id (fused) vs 151936 fp32 logits (GEMV only)"
    return out


def bench_single_gemv(lin, torch, dev, stream, N=6144, K=2048, reps=10):
    """One W8A32 decode GEMV, x fp32 [1, K], W int8 [N, K] with per-row
    scales: the launches over 41+ distinct weight copies (>= 512 MB, beyond
    the 256 MB Infinity Cache) captured in one HIP graph and replayed."""
    copies = max(41, int(np.ceil(512e6 / (N * K))))
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    Ws = []
    for _ in range(copies):
        w = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
        Ws.append(lin.DeviceWeights.from_codes(w, torch.rand(N, device=dev, generator=g) * 0.018 + 0.002))
        del w
    x = torch.randn((1, K), device=dev, generator=g)
    y = torch.empty((1, N), device=dev)
    with torch.cuda.stream(stream):
        for W in Ws:
            lin.w8a32_linear_dev(x, W, y, stream=stream)
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for W in Ws:
            lin.w8a32_linear_dev(x, W, y, stream=stream)
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) * 1e-3 / (reps * copies)
    b = gemv_bytes(N, K)
    del graph
    for W in Ws:
        W.close()
    return {"N": N, "K": K, "us": round(t * 1e6, 3), "GBps": round(b / t / 1e9, 1),
            "frac_hbm": round(b / t / 1e9 / HBM_PEAK_GBS, 4), "bytes": b, "weight_copies": copies,
            "timing": "graph of one launch per weight copy, replayed; HIP events; per-launch average"}


def bench_w8a8_prefill(lin, torch, dev):
    """W8A8 prefill GEMMs at M = 1024 (N = 6144, K = 2048 and N = 2048, K =
    6144), weights rotating over >= 512 MB of copies, graph-replayed calls:
    the whole call (per-token quantization into int8 tiles + the int8 MFMA
    GEMM, tl_w8a8_linear_f32_dev), and its two halves timed on their own
    (tl_w8a8_quantize_tiles_dev; tl_w8a8_linear_tiles_dev, the GEMM alone on
    codes quantized once)."""
    lib = lin.load_library()
    out = {}
    tot_ops, tot_t, tot_g = 0.0, 0.0, 0.0
    for (N, K) in [(6144, 2048), (2048, 6144)]:
        M = 1024
        Ws = rotating(lin, torch, dev, N, K, min_bytes=512e6)
        x = torch.randn((M, K), device=dev)
        y = torch.empty((M, N), device=dev)
        tiles = torch.empty(lib.tl_w8a8_tiles_bytes(M, K), dtype=torch.uint8, device=dev)
        scales = torch.empty(-(-M // 16) * 16, dtype=torch.float32, device=dev)
        t = time_graph(torch, lambda i, st: lin.w8a8_linear_f32_dev(x, Ws[i], y, stream=st), len(Ws))
        tq = time_graph(torch, lambda i, st: lin.w8a8_quantize_tiles_dev(x, tiles, scales, stream=st), 1)
        lin.w8a8_quantize_tiles_dev(x, tiles, scales)
        tg = time_graph(torch, lambda i, st: lin.w8a8_linear_tiles_dev(tiles, scales, Ws[i], y, stream=st), len(Ws))
        ops = 2.0 * M * N * K
        qbytes = M * K * 4 + M * K + M * 4
        out[f"M{M}_N{N}_K{K}"] = {"us": round(t * 1e6, 2), "tops": round(ops / t / 1e12, 1),
                                   "frac_int8_peak": round(ops / t / 1e12 / INT8_PEAK_TOPS, 4),
                                   "gemm_us": round(tg * 1e6, 2),
                                   "gemm_frac_int8_peak": round(ops / tg / 1e12 / INT8_PEAK_TOPS, 4),
                                   "quantize_us": round(tq * 1e6, 2),
                                   "quantize_GBps": round(qbytes / tq / 1e9, 1)}
        tot_ops += ops
        tot_t += t
        tot_g += tg
        for W in Ws:
            W.close()
    out["tops"] = round(tot_ops / tot_t / 1e12, 1)
    out["frac_int8_peak"] = round(tot_ops / tot_t / 1e12 / INT8_PEAK_TOPS, 4)
    out["gemm_frac_int8_peak"] = round(tot_ops / tot_g / 1e12 / INT8_PEAK_TOPS, 4)
    out["includes"] = ("us / frac_int8_peak: per-token activation quantization kernel + int8 MFMA GEMM, fp32 "
                       "in/out; gemm_us: the GEMM alone on tiled codes; quantize_us: the quantization alone "
                       "(fp32 rows read, int8 tiles and scales written); graph-replayed calls")
    return out


def bench_decoder_generate(lin, torch, dev, n_layers=28, vocab=151936, prefix=1200, steps=512):
    """The full-decoder workload: 28 layers, a `prefix`-token prefill
    (decoder_prefill_step, timed with W8A8 and with fp32-activation linears)
    then `steps` greedy decode steps on the device
    (graph replays of 28 x 6 layer launches + lm_head + token/embedding
    step).  Random int8 weights per row-scaled projection, a random fp32
    embedding table, lm_head over the full vocabulary; the prompt is the
    embeddings of random token ids."""
    import ctypes
    lib = lin.load_library()
    rng = np.random.default_rng(5)
    H, KV, FF, HD = 2048, 1024, 6144, 128
    max_seq = 2048
    model = lib.decoder_model_alloc()
    cache = lib.decoder_cache_alloc(max_seq)
    scratch = lib.decoder_scratch_alloc_fn(max_seq)
    f32p = ctypes.POINTER(ctypes.c_float)
    i8p = ctypes.POINTER(ctypes.c_int8)

    def mat(n, k):
        w = rng.integers(-127, 128, (n, k), dtype=np.int8)
        s = rng.uniform(1e-4, 5e-4, n).astype(np.float32)   # keeps activations O(1)
        return w, s

    def vec(n):
        return (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    for l in range(n_layers):
        mats = [mat(H, H), mat(KV, H), mat(KV, H), mat(H, H), mat(FF, H), mat(FF, H), mat(H, FF)]
        norms = [vec(H), vec(H), vec(HD), vec(HD)]
        args = []
        for w, s in mats:
            args += [w.ctypes.data_as(i8p), s.ctypes.data_as(f32p)]
        args += [n.ctypes.data_as(f32p) for n in norms]
        lib.decoder_set_layer_weights(model, l, *args)
        lin.check(lib, "decoder_set_layer_weights")
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    lm_w = torch.randint(-127, 128, (vocab, H), dtype=torch.int8, device=dev, generator=gen)
    lm_s = torch.rand(vocab, device=dev, generator=gen) * 4e-4 + 1e-4
    lm = lin.DeviceWeights.from_codes(lm_w, lm_s)
    del lm_w
    embed = torch.randn((vocab, H), device=dev, generator=gen)
    fnorm = vec(H)
    half = HD // 2
    cos = np.empty((max_seq, half), np.float32)
    sin = np.empty((max_seq, half), np.float32)
    lib.decoder_precompute_rope(cos.ctypes.data_as(f32p), sin.ctypes.data_as(f32p), max_seq, HD,
                                (ctypes.c_int * 3)(24, 20, 20), (ctypes.c_float * 3)(5e6, 5e6, 5e6))

    def generate(first, n):
        toks = np.empty(n, np.int32)
        rc = lib.tl_decoder_generate(model, cache, scratch, lm.handle, fnorm.ctypes.data_as(f32p),
                                     embed.data_ptr(), int(first), int(n),
                                     toks.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                                     cos.ctypes.data_as(f32p), sin.ctypes.data_as(f32p))
        if rc != 0:
            lin.check(lib, "tl_decoder_generate")
        return toks

    # warm-up: a full-size prefill in each mode (work-space growth: activation
    # buffers, pinned row staging) and a few steps (graph capture)
    ids = rng.integers(0, vocab, prefix)
    hidden0 = embed[torch.from_numpy(ids).to(dev)].cpu().numpy()
    lib.decoder_cache_clear(cache)
    for w8 in (1, 0):
        hw = np.array(hidden0, copy=True)
        lib.tl_decoder_set_prefill_w8a8(model, w8)
        lib.decoder_cache_clear(cache)
        lib.decoder_prefill_step(model, cache, hw.ctypes.data_as(f32p), scratch, cos.ctypes.data_as(f32p),
                                 sin.ctypes.data_as(f32p), prefix)
        lin.check(lib, "decoder_prefill_step")
    generate(1, 4)
    # the workload: prefill `prefix` tokens, greedy token from the last row, `steps` decode steps.
    # The prefill runs twice: W8A8 linears (the workload's prefill), then the
    # reference decoder's fp32-activation linears, whose cache the decode uses.
    def prefill(w8a8):
        lib.tl_decoder_set_prefill_w8a8(model, w8a8)
        lib.decoder_cache_clear(cache)
        hh = np.array(hidden0, copy=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        lib.decoder_prefill_step(model, cache, hh.ctypes.data_as(f32p), scratch, cos.ctypes.data_as(f32p),
                                 sin.ctypes.data_as(f32p), prefix)
        lin.check(lib, "decoder_prefill_step")
        return hh, time.perf_counter() - t0
    _, t_pre8 = prefill(1)
    h, t_pre = prefill(0)
    lm_logits_tok = torch.empty(1, dtype=torch.int32, device=dev)
    lin.lm_head_argmax_dev(torch.from_numpy(h[-1].copy()).to(dev), torch.from_numpy(fnorm).to(dev), lm,
                           lm_logits_tok)
    first = int(lm_logits_tok.cpu().numpy()[0])
    t0 = time.perf_counter()
    toks2 = generate(first, steps)
    t = time.perf_counter() - t0
    out = {"tok_s": round(steps / t, 1), "ms_per_token": round(t / steps * 1e3, 4),
           "layers": n_layers, "vocab": vocab, "cache_len_start": prefix, "steps": steps,
           "launches_per_token": n_layers * 5 + 2,
           "prefill_tokens": prefix,
           "prefill_w8a8_ms": round(t_pre8 * 1e3, 3), "prefill_w8a8_tok_s": round(prefix / t_pre8, 1),
           "prefill_w8a32_ms": round(t_pre * 1e3, 3), "prefill_w8a32_tok_s": round(prefix / t_pre, 1),
           "end_to_end_s": round(t_pre8 + t, 4),
           "distinct_tokens": int(len(set(toks2.tolist()))),
           "tokens_sha1": hashlib.sha1(toks2.tobytes()).hexdigest()[:16],
           "timing": "host wall clock: the prefill call (hidden rows in and out over PCIe included), "
                     "then the graph-replayed decode steps + the tokens' device-to-host copy"}
    lm.close()
    lib.decoder_model_free(model)
    lib.decoder_cache_free(cache)
    lib.decoder_scratch_free_fn(scratch)
    return out


def host_cores():
    """Threads for the CPU baseline: every core this process may run on
    (its affinity mask), capped by OMP_NUM_THREADS when the host sets it (the
    GPU box gives one GPU's process a 16-core share and sets it to 16)."""
    try:
        n = len(os.sched_getaffinity(0))
    except Exception:
        n = os.cpu_count() or 1
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def host_description():
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        aff = len(os.sched_getaffinity(0))
    except Exception:
        aff = None
    return {"host_cpu": model, "nproc": os.cpu_count(), "affinity_cpus": aff,
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def cpu_baseline(seconds=10.0, legs_seconds=20.0):
    """The oracle's M=1 GEMV (same formula as the reference's w8a32_gemv,
    OpenMP over row chunks like its GCD fan-out) on the host cores, over the
    same steps as the GPU: one layer's projection set (layer copy i % 28 of
    28 distinct ones) + the lm_head (one of two copies, alternating; 2.0 GB
    of int8 weights in all, so no cache holds them).  Steps are timed until
    the time budget is spent; the median step time gives GB/s.  Beside it,
    the reference's M>1 decompositions on the same cores (oracle/baseline.c:
    dequantized 64/128-row weight tiles and a blocked fp32 SGEMM): W8A8 at
    M=1024, the W8A16 sweep and w8a32_linear at the 1200-token prefill."""
    from oracle import oracle as orc
    native = True
    try:
        orc.build(native=True)
    except Exception:
        native = False
    cores = host_cores()
    rng = np.random.default_rng(0)
    # two lm_head copies, alternating: a host last-level cache must not hold
    # the lm_head from one step to the next
    shapes = [(f"l{l}.{n}", N, K) for l in range(LAYERS) for (n, N, K) in LAYER_SHAPES] + [LM_HEAD, LM_HEAD]
    mats = []
    for (name, N, K) in shapes:
        w = rng.integers(-127, 128, (N, K), dtype=np.int8)
        s = rng.uniform(0.002, 0.02, N).astype(np.float32)
        x = rng.standard_normal(K, dtype=np.float32)
        mats.append((w, s, x, np.empty(N, np.float32)))
    nl = len(LAYER_SHAPES)
    for (w, s, x, y) in mats[:4]:
        orc.w8a32_gemv_timed(x, w, s, y, cores, native=native)        # warm-up
    times = []
    t_end = time.perf_counter() + seconds
    i = 0
    while time.perf_counter() < t_end or len(times) < 2:
        step = mats[nl * (i % LAYERS):nl * (i % LAYERS) + nl] + [mats[-1 - (i % 2)]]
        t0 = time.perf_counter()
        for (w, s, x, y) in step:
            orc.w8a32_gemv_timed(x, w, s, y, cores, native=native)
        times.append(time.perf_counter() - t0)
        i += 1
    t_step = float(np.median(times))
    del mats
    step_bytes = sum(gemv_bytes(N, K) for (_, N, K) in LAYER_SHAPES + [LM_HEAD])
    out = {"value": round(step_bytes / t_step / 1e9, 2), "unit": "GB/s", "cores": cores, "kind": "port",
           "ms_per_step": round(t_step * 1e3, 3), "steps_timed": len(times)}
    out.update(host_description())
    out["sample"] = (f"oracle M=1 GEMV ({'-march=native' if native else 'x86-64-v3'}, OpenMP, {cores} threads) "
                     f"over the benchmark's steps (one layer's projection set of 28 distinct copies + one of two "
                     f"lm_head copies, 361.5 MB per step), median of {len(times)} steps in ~{seconds:.0f} s")

    # ---- the M>1 legs: each point timed on distinct weights, median of its calls
    budget_end = time.perf_counter() + legs_seconds

    def timed(fn, calls):
        fn()                                          # warm-up (first touch, tile buffers)
        ts = []
        for _ in range(calls):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts))

    legs = {}
    w8 = {}
    for (N, K) in [(6144, 2048), (2048, 6144)]:
        M = 1024
        x = rng.standard_normal((M, K), dtype=np.float32)
        xq, xs = orc.quantize_rows(x)
        w = rng.integers(-127, 128, (N, K), dtype=np.int8)
        s = rng.uniform(0.002, 0.02, N).astype(np.float32)
        t = timed(lambda: orc.base_w8a8_gemm(xq, xs, w, s, cores, native), 2)
        w8[f"M{M}_N{N}_K{K}"] = {"ms": round(t * 1e3, 2), "GOPS": round(2.0 * M * N * K / t / 1e9, 1)}
    legs["w8a8_m1024"] = w8
    sw = {}
    K = 2048
    for N in (2048, 4096, 12288):
        w = rng.integers(-127, 128, (N, K), dtype=np.int8)
        s = rng.uniform(0.002, 0.02, N).astype(np.float32)
        for M in (1, 8, 64, 256, 1024):
            if time.perf_counter() > budget_end:
                break
            xb = (rng.standard_normal((M, K), dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)
            t = timed(lambda: orc.base_w8a16_linear(xb, w, s, cores, native), 5 if M <= 64 else 2)
            b = N * K + 4 * N + 2 * M * K + 2 * M * N
            sw[f"M{M}_N{N}"] = {"ms": round(t * 1e3, 3), "GFLOPS": round(2.0 * M * N * K / t / 1e9, 1),
                                "GBps": round(b / t / 1e9, 1)}
    legs["w8a16_sweep"] = sw
    pre = {}
    tot = 0.0
    for (name, N, K) in LAYER_SHAPES:
        if time.perf_counter() > budget_end:
            break
        M = 1200
        x = rng.standard_normal((M, K), dtype=np.float32)
        w = rng.integers(-127, 128, (N, K), dtype=np.int8)
        s = rng.uniform(0.002, 0.02, N).astype(np.float32)
        t = timed(lambda: orc.base_w8a32_gemm(x, w, s, cores, native), 1)
        pre[name] = {"ms": round(t * 1e3, 2), "GFLOPS": round(2.0 * M * N * K / t / 1e9, 1)}
        tot += t
    if len(pre) == len(LAYER_SHAPES):
        pre["layer_ms"] = round(tot * 1e3, 2)
    legs["w8a32_prefill_m1200"] = pre
    legs["kind"] = "port: the reference's tile decompositions (oracle/baseline.c), blocked fp32 SGEMM"
    out["m_gt_1_legs"] = legs
    return out


def rotating(lin, torch, dev, N, K, min_bytes=600e6):
    copies = max(2, int(np.ceil(min_bytes / (N * K))))
    Ws = []
    for _ in range(copies):
        w = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev)
        s = torch.rand(N, device=dev) * 0.018 + 0.002
        Ws.append(lin.DeviceWeights.from_codes(w, s))
    return Ws


def time_calls(torch, fn, n_w, reps=20, rounds=3):
    """Per-call time of fn(i % n_w, stream): the median over `rounds` timed
    rounds of `reps` back-to-back calls (HIP events), after warm-up calls on
    every weight copy."""
    st = torch.cuda.current_stream()
    for i in range(max(3, n_w)):
        fn(i % n_w, st)
    torch.cuda.synchronize()
    ts = []
    for r in range(rounds):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        for i in range(reps):
            fn((r * reps + i) % n_w, st)
        e1.record(st)
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1) * 1e-3 / reps)
    return float(np.median(ts))


def time_graph(torch, fn, n_w, min_calls=40, rounds=3):
    """Per-call time of fn(i % n_w, stream) with the calls captured back to
    back in one HIP graph (max(n_w, min_calls) calls: every weight copy once
    or more) and replayed: the kernels' own time, without the host's launch
    gaps (eager calls from Python are launch-bound below about 5 us).  Warm-up
    calls first, so every work-space exists before the capture; the median
    over `rounds` replays."""
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        for i in range(max(3, n_w)):
            fn(i % n_w, st)
    st.synchronize()
    calls = max(n_w, min_calls)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        for i in range(calls):
            fn(i % n_w, st)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(rounds):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1) * 1e-3 / calls)
    del g
    return float(np.median(ts))


def read_floor(lin, torch, dev, nbytes, min_bytes=640e6):
    """The launch-time floor of reading `nbytes` once: tl_stream_read_dev (a
    grid-stride read with the GEMV's non-temporal 16-byte loads and nothing
    else) over rotating buffers (> 640 MB, past the 256 MB MALL), graph-replayed,
    best over grids of 256..2048 work-groups and 4 or 8 loads in flight."""
    lib = lin.load_library()
    n = (int(nbytes) + 15) // 16 * 16
    copies = max(2, int(np.ceil(min_bytes / n)))
    bufs = [torch.empty(n, dtype=torch.uint8, device=dev).fill_(1) for _ in range(copies)]
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    best = None
    for u in (4, 8):
        for grid in (256, 512, 1024, 2048):
            if grid * 256 * u * 16 > n:
                continue

            def fn(i, st, grid=grid, u=u):
                rc = lib.tl_stream_read_dev(bufs[i].data_ptr(), n, grid, u, sink.data_ptr(), st.cuda_stream)
                assert rc == 0, lin.check(lib, "tl_stream_read_dev")
            t = time_graph(torch, fn, copies)
            if best is None or t < best[0]:
                best = (t, grid, u)
    if best is None:          # fewer bytes than one full pass of 256 work-groups
        def fn(i, st):
            rc = lib.tl_stream_read_dev(bufs[i].data_ptr(), n, 256, 4, sink.data_ptr(), st.cuda_stream)
            assert rc == 0, lin.check(lib, "tl_stream_read_dev")
        best = (time_graph(torch, fn, copies), 256, 4)
    del bufs
    t, grid, u = best
    return {"bytes": n, "us": round(t * 1e6, 2), "GBps": round(n / t / 1e9, 1),
            "frac_hbm": round(n / t / 1e9 / HBM_PEAK_GBS, 4), "grid": grid, "u": u}


def bench_decode_rows(lin, torch, dev):
    """W8A32 decode rows M = 1, 2, 4, 8 (M = 1: int8 GEMV; M = 2..8: fp32
    semantics, int8 digit planes on the MFMA) per decode shape, HBM GB/s;
    graph-replayed calls (time_graph)."""
    out = {}
    for (name, N, K) in LAYER_SHAPES + [LM_HEAD]:
        Ws = rotating(lin, torch, dev, N, K)
        row = {}
        for M in (1, 2, 4, 8):
            x = torch.randn((M, K), device=dev)
            y = torch.empty((M, N), device=dev)
            t = time_graph(torch, lambda i, st: lin.w8a32_linear_dev(x, Ws[i], y, stream=st), len(Ws))
            b = N * K + 4 * N + 4 * M * K + 4 * M * N
            row[f"M{M}"] = {"us": round(t * 1e6, 2), "GBps": round(b / t / 1e9, 1),
                            "frac_hbm": round(b / t / 1e9 / HBM_PEAK_GBS, 4)}
        out[f"{name}_{N}x{K}"] = row
        for W in Ws:
            W.close()
    return out


REFERENCE_W8A32_ROWS = [("q_proj", 2048, 2048, 1), ("k_proj", 256, 2048, 1), ("v_proj", 256, 2048, 1),
                        ("o_proj", 2048, 2048, 1), ("gate_proj", 6144, 2048, 1), ("up_proj", 6144, 2048, 1),
                        ("down_proj", 2048, 6144, 1), ("q_proj", 2048, 2048, 32), ("gate_proj", 6144, 2048, 32),
                        ("down_proj", 2048, 6144, 32)]


def bench_reference_w8a32_rows(lin, torch, dev):
    """The reference benchmark's own W8A32 rows (bench_flops.py:257-268: the
    separate decode projections at batch 1, and q, gate and down at batch 32),
    graph-replayed over >= 600 MB of rotating weights; GFLOPS = 2 M N K / t
    as the reference reports them, and HBM GB/s of the rows' bytes."""
    out = {}
    for (name, N, K, M) in REFERENCE_W8A32_ROWS:
        Ws = rotating(lin, torch, dev, N, K)
        x = torch.randn((M, K), device=dev)
        y = torch.empty((M, N), device=dev)
        t = time_graph(torch, lambda i, st: lin.w8a32_linear_dev(x, Ws[i], y, stream=st), len(Ws))
        b = N * K + 4 * N + 4 * M * K + 4 * M * N
        out[f"{name}_{N}x{K}_batch{M}"] = {"us": round(t * 1e6, 2), "GFLOPS": round(2.0 * M * N * K / t / 1e9, 1),
                                          "GBps": round(b / t / 1e9, 1),
                                          "frac_hbm": round(b / t / 1e9 / HBM_PEAK_GBS, 4)}
        for W in Ws:
            W.close()
    return out


def bench_w8a16_sweep(lin, torch, dev):
    """W8A16 sweep: bf16 X [M, 2048], int8 W [N, 2048], bf16 out; graph-replayed
    calls (time_graph)."""
    out = {}
    K = 2048
    for N in (2048, 4096, 12288):
        Ws = rotating(lin, torch, dev, N, K)
        for M in (1, 8, 64, 256, 1024):
            x = torch.randn((M, K), device=dev).to(torch.bfloat16)
            y = torch.empty((M, N), device=dev, dtype=torch.bfloat16)
            t = time_graph(torch, lambda i, st: lin.w8a16_linear_dev(x, Ws[i], y, stream=st), len(Ws))
            ops = 2.0 * M * N * K
            b = N * K + 4 * N + 2 * M * K + 2 * M * N
            hbm = M <= 64
            frac = (b / t / 1e9 / HBM_PEAK_GBS) if hbm else (ops / t / 1e12 / BF16_PEAK_TFLOPS)
            out[f"M{M}_N{N}"] = {"us": round(t * 1e6, 2), "TFLOPs": round(ops / t / 1e12, 1),
                                 "GBps": round(b / t / 1e9, 1), "bound": "hbm" if hbm else "mfma",
                                 "frac": round(frac, 4)}
        for W in Ws:
            W.close()
    return out


def bench_w8a32_prefill(lin, torch, dev, M=1200):
    """The reference decoder's prefill linear path, w8a32_linear(batch=S)
    (fp32 X times dequantized weights), at S = 1200 on the fused layer shapes;
    computed fp32-accurately on the int8 MFMA, each token split into four int8
    planes (the plane split launch included)."""
    out = {}
    tot_f, tot_t = 0.0, 0.0
    for (name, N, K) in LAYER_SHAPES:
        Ws = rotating(lin, torch, dev, N, K, min_bytes=300e6)
        x = torch.randn((M, K), device=dev)
        y = torch.empty((M, N), device=dev)
        t = time_calls(torch, lambda i, st: lin.w8a32_linear_dev(x, Ws[i], y, stream=st), len(Ws), reps=10)
        f = 2.0 * M * N * K
        out[name] = {"us": round(t * 1e6, 1), "TFLOPs_fp32_equiv": round(f / t / 1e12, 1)}
        tot_f += f
        tot_t += t
        for W in Ws:
            W.close()
    out["layer_ms"] = round(tot_t * 1e3, 3)
    out["prefill_tok_s_linear_only"] = round(M / (LAYERS * tot_t), 1)
    return out


def bench_host_abi(lin, reps=200):
    """The reference's own entry point, w8a32_linear(batch=1) on host
    pointers: registered weights, x copied in and y copied out through pinned
    staging on every call, stream synchronised before return.  Wall-clock per
    call (PCIe and synchronisation included)."""
    lib = lin.load_library()
    rng = np.random.default_rng(1)
    out = {}
    for (name, N, K) in [("qkv", 4096, 2048), ("lm_head", 151936, 2048)]:
        w = rng.integers(-127, 128, (N, K), dtype=np.int8)
        s = rng.uniform(0.002, 0.02, N).astype(np.float32)
        x = rng.standard_normal((1, K), dtype=np.float32)
        y = np.empty((1, N), np.float32)
        if lib.tl_register_weights(lin._p(w, lin.ctypes.c_int8), lin._p(s, lin.ctypes.c_float), N, K) != 0:
            lin.check(lib, "tl_register_weights")
        n = reps if N < 100000 else max(20, reps // 10)
        for _ in range(20):
            lin.w8a32_linear(x, w, s, out=y)
        # median per-call wall time (robust against the driver's deferred work
        # after the decode set's 1.72 GB are freed just before)
        ts = []
        for _ in range(n):
            t0 = time.perf_counter()
            lin.w8a32_linear(x, w, s, out=y)
            ts.append(time.perf_counter() - t0)
        t = float(np.median(ts))
        b = gemv_bytes(N, K)
        out[f"{name}_{N}x{K}"] = {"us": round(t * 1e6, 2), "GBps": round(b / t / 1e9, 1)}
        lib.tl_evict_weights(lin._p(w, lin.ctypes.c_int8))
    # the same QKV call from 1 and from 4 threads (one ctypes call each, which
    # releases the interpreter lock; every thread on its own weights)
    import threading
    calls, keep = [], []
    for _ in range(4):
        N, K = 4096, 2048
        w = rng.integers(-127, 128, (N, K), dtype=np.int8)
        s = rng.uniform(0.002, 0.02, N).astype(np.float32)
        x = rng.standard_normal((1, K), dtype=np.float32)
        y = np.empty((1, N), np.float32)
        keep.append((w, s, x, y))
        calls.append((lin._p(x, lin.ctypes.c_float), lin._p(w, lin.ctypes.c_int8), lin._p(s, lin.ctypes.c_float),
                      lin._p(y, lin.ctypes.c_float), N, K))

    def work(c, n):
        xp, wp, sp, yp, N, K = c
        for _ in range(n):
            lib.w8a32_linear(xp, wp, sp, None, yp, None, 1, N, K)

    for c in calls:
        work(c, 10)
    n = 1000
    t0 = time.perf_counter()
    for c in calls:
        work(c, n)
    t1 = (time.perf_counter() - t0) / (4 * n)
    ths = [threading.Thread(target=work, args=(c, n)) for c in calls]
    t0 = time.perf_counter()
    for th in ths:
        th.start()
    for th in ths:
        th.join()
    t4 = (time.perf_counter() - t0) / (4 * n)
    for (w, *_r) in keep:
        lib.tl_evict_weights(lin._p(w, lin.ctypes.c_int8))
    out["qkv_threads"] = {"threads1_us_per_call": round(t1 * 1e6, 2), "threads4_us_per_call": round(t4 * 1e6, 2),
                          "speedup": round(t1 / t4, 2)}
    out["includes"] = ("median per call: host x -> HBM, GEMV, HBM -> host y, stream sync; "
                       "weights already resident; qkv_threads: aggregate time per call of 4000 calls "
                       "from 1 thread and from 4 threads")
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-prefill", action="store_true", help="skip the W8A8 prefill timing")
    ap.add_argument("--quick", action="store_true",
                    help="decode set only (no prefill, sweeps or CPU baseline)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the W8A8 prefill timing (for counter runs)")
    ap.add_argument("--w8a16-only", action="store_true",
                    help="only the W8A16 sweep (for counter runs)")
    ap.add_argument("--decoder-layers", type=int, default=28,
                    help="layers of the full-decoder workload (fewer only to profile it)")
    ap.add_argument("--decoder-steps", type=int, default=512,
                    help="greedy steps of the full-decoder workload (fewer only to profile it)")
    ap.add_argument("--decoder-only", action="store_true",
                    help="only the device-resident 28-layer greedy decoder timing")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="run a 512 MiB device copy (counter calibration) and one eager decode "
                         "step, then exit; used under rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE")
    ap.add_argument("--summarize-trace", metavar="CSV",
                    help="write the timed steps' summary of a rocprofv3 kernel_trace.csv of this "
                         "benchmark (run with the same --steps) to stdout, then exit (no GPU use)")
    ap.add_argument("--trace-command", default="",
                    help="the profiling command, recorded in the --summarize-trace output")
    args = ap.parse_args()
    if args.summarize_trace:
        print(summarize_trace(args.summarize_trace, args.steps, args.trace_command))
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1"}))
        sys.exit(2)
    rank = int(os.environ.get("RANK", "0"))

    import torch
    import __graft_entry__ as ge
    ge.load_package()
    import importlib
    lin = importlib.import_module("typhoon_ocr_server_amd.linear")
    lin.load_library()
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU")
    dev = torch.device("cuda:0")

    if args.prefill_only:
        print(json.dumps({"w8a8_prefill": bench_w8a8_prefill(lin, torch, dev)}), flush=True)
        return
    if args.w8a16_only:
        print(json.dumps({"w8a16_sweep": bench_w8a16_sweep(lin, torch, dev)}), flush=True)
        return
    if args.decoder_only:
        print(json.dumps({"decoder_greedy": bench_decoder_generate(lin, torch, dev, n_layers=args.decoder_layers,
                                                                   steps=args.decoder_steps)}), flush=True)
        return
    log("building the decode set (1.72 GB of layer weights, two 311 MB lm_head copies)")
    items = build_decode_set(lin, torch, dev)
    nl = len(LAYER_SHAPES)
    layers = [items[nl * l:nl * l + nl] for l in range(LAYERS)]
    lm_heads = items[nl * LAYERS:]

    # the benchmark's step i: layer copy i % 28's projection set + lm_head copy i % 2
    def step_items(i):
        return layers[i % LAYERS] + [lm_heads[i % LM_COPIES]]

    seq = [it for i in range(LAYERS) for it in step_items(i)]
    if args.traffic_probe:
        src = torch.empty(COPY_PROBE_BYTES // 4, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        st = torch.cuda.current_stream()
        run_step(lin, seq, st)
        torch.cuda.synchronize()
        log("traffic probe done")
        return
    step_bytes = sum(gemv_bytes(N, K) for (_, N, K) in LAYER_SHAPES + [LM_HEAD])
    stream = torch.cuda.Stream()
    marker = TraceMarker(lin, torch, dev)

    def capture(its):
        with torch.cuda.stream(stream):
            for _ in range(max(1, args.warmup)):
                run_step(lin, its, stream)
        stream.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            run_step(lin, its, stream)
        torch.cuda.synchronize()
        for _ in range(args.warmup):
            g.replay()
        torch.cuda.synchronize()
        return g

    def time_replays(g, reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e-3 / reps, time.perf_counter() - t0

    # The timed steps run as the decoder runs its layers: captured back to
    # back in one HIP graph, so a step pays kernel boundaries only, not a graph
    # launch of its own.  The same steps as one graph each are timed beside it
    # (graph_per_step).
    log(f"warm-up (eager) and graph capture: {args.steps} steps in one graph")
    with torch.cuda.stream(stream):
        for i in range(LAYERS):
            run_step(lin, step_items(i), stream)
    stream.synchronize()
    g_steps = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_steps, stream=stream):
        for i in range(args.steps):
            run_step(lin, step_items(i), stream)
    g_warm = None
    if args.warmup > 0:
        g_warm = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_warm, stream=stream):
            for i in range(args.warmup):
                run_step(lin, step_items(i), stream)
    torch.cuda.synchronize()
    if g_warm is not None:
        g_warm.replay()
    torch.cuda.synchronize()
    # TIMED_REPLAYS replays of the K-step graph, each timed on its own (HIP
    # events on the replay stream, synchronised before and after); the median
    # is the figure.  A marker launch (outside the events) brackets every timed
    # replay, so a kernel trace of this run can find the timed launches.
    log(f"timing {args.steps} steps, {TIMED_REPLAYS} replays")
    t_reps, wall = [], 0.0
    replay_stream = torch.cuda.current_stream()      # CUDAGraph.replay() launches on the current stream
    for _ in range(TIMED_REPLAYS):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        marker.launch(replay_stream)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record(replay_stream)
        g_steps.replay()
        e1.record(replay_stream)
        torch.cuda.synchronize()
        wall += time.perf_counter() - t0
        marker.launch(replay_stream)
        torch.cuda.synchronize()
        t_reps.append(e0.elapsed_time(e1) * 1e-3 / args.steps)
    t_step = float(np.median(t_reps))
    value = step_bytes / t_step / 1e9
    del g_steps, g_warm

    log("the same steps as one graph launch each")
    graphs = [capture(step_items(i)) for i in range(LAYERS)]
    t_gs = []
    for _ in range(3):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for i in range(args.steps):
            graphs[i % LAYERS].replay()
        e1.record()
        torch.cuda.synchronize()
        t_gs.append(e0.elapsed_time(e1) * 1e-3 / args.steps)
    t_step_graphs = float(np.median(t_gs))
    graph_per_step = {"ms_per_step": round(t_step_graphs * 1e3, 5),
                      "GBps": round(step_bytes / t_step_graphs / 1e9, 1),
                      "frac_hbm": round(step_bytes / t_step_graphs / 1e9 / HBM_PEAK_GBS, 4),
                      "timing": "one graph launch per step, median of 3 rounds of --steps steps"}
    del graphs

    log("the full decoder step: 28 layers + lm_head in one graph")
    full = [it for l in layers for it in l] + [lm_heads[0]]
    graph28 = capture(full)
    t28, _ = time_replays(graph28, max(5, args.steps // 5))
    bytes28 = sum(gemv_bytes(N, K) for (_, N, K, *_r) in full)
    step28 = {"ms": round(t28 * 1e3, 4), "GBps": round(bytes28 / t28 / 1e9, 1),
              "frac_hbm": round(bytes28 / t28 / 1e9 / HBM_PEAK_GBS, 4), "launches": len(full),
              "bytes": bytes28, "tok_s_linear_layers": round(1.0 / t28, 1)}
    del graph28

    log("per-shape launch timing (graph replay)")
    per = time_shapes(lin, torch, items, dev)
    per_shape = {}
    for key, (N, K, t) in per.items():
        b = gemv_bytes(N, K)
        per_shape[key] = {"N": N, "K": K, "us": round(t * 1e6, 2), "GBps": round(b / t / 1e9, 1),
                          "frac_hbm": round(b / t / 1e9 / HBM_PEAK_GBS, 4)}
    if not args.quick:
        # what a launch that only reads the same bytes takes on this device
        log("read floor per shape (plain streaming read of the same bytes)")
        for key, (N, K, t) in per.items():
            f = read_floor(lin, torch, dev, gemv_bytes(N, K))
            per_shape[key]["read_floor_us"] = f["us"]
            per_shape[key]["read_floor_frac_hbm"] = f["frac_hbm"]
            per_shape[key]["vs_read_floor"] = round(f["us"] * 1e-6 / t, 4)
    # Every launch of a step is the GEMV kernel.  `achieved` is the step's
    # algorithmic bytes over the GEMV kernel time of a step in the committed
    # rocprofv3 kernel trace of this command (the timed replays' launches,
    # End - Start summed per step), while that trace was taken on the current
    # GEMV sources; `live` is the same ratio on this run's HIP-event step time
    # (launch gaps included).
    n_per_step = len(LAYER_SHAPES) + 1
    avg_bytes = step_bytes / n_per_step
    live_achieved = step_bytes / t_step / 1e9
    live = {"achieved": round(live_achieved, 1), "frac": round(live_achieved / HBM_PEAK_GBS, 4),
            "avg_launch_us": round(t_step / n_per_step * 1e6, 3),
            "replay_ms_per_step": [round(t * 1e3, 5) for t in t_reps],
            "source": f"HIP events on the replay stream, median of {TIMED_REPLAYS} replays of the "
                      f"{args.steps}-step graph, step time / {n_per_step} launches"}
    prof_us, prof_note = profiled_step_kernel_us(args.steps)
    if prof_us is not None:
        achieved = step_bytes / (prof_us * 1e-6) / 1e9
        avg_launch_us = prof_us / n_per_step
        src = f"rocprofv3 kernel trace of this command ({TRACE_SUMMARY.relative_to(ROOT)}): {prof_note}"
    else:
        achieved, avg_launch_us = live_achieved, t_step / n_per_step * 1e6
        src = f"HIP events of this run ({prof_note})"
    traffic, traffic_note = measured_traffic()
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": traffic_note,
                "kernel": f"gemv_i8_kernel (all {n_per_step} launches of a step)",
                "bytes_per_launch": round(avg_bytes), "avg_launch_us": round(avg_launch_us, 3),
                "achieved_source": src, "live": live, "per_shape": per_shape}

    log("fused greedy lm_head step")
    greedy = bench_lm_head_greedy(lin, torch, items[-1][3], items[-1][2], dev, stream)

    # the decode set's 1.72 GB is no longer needed
    for it in items:
        it[3].close()
    del items

    log("single decode GEMV 6144x2048 over 41 weight copies")
    single = bench_single_gemv(lin, torch, dev, stream)

    prefill = rows = ref_rows = sweep = pre32 = host = None
    if not args.quick:
        log("host-pointer ABI (PCIe-inclusive)")
        host = bench_host_abi(lin)
    if not args.no_prefill and not args.quick:
        log("W8A8 prefill timing")
        prefill = bench_w8a8_prefill(lin, torch, dev)
        log("W8A32 decode rows M=1..8")
        rows = bench_decode_rows(lin, torch, dev)
        log("W8A32: the reference benchmark's rows (batch 1 and 32)")
        ref_rows = bench_reference_w8a32_rows(lin, torch, dev)
        log("W8A16 sweep")
        sweep = bench_w8a16_sweep(lin, torch, dev)
        log("W8A32 prefill (fp32 semantics)")
        pre32 = bench_w8a32_prefill(lin, torch, dev)

    dec = None
    if not args.quick:
        log("device-resident greedy decoder (28 layers)")
        dec = bench_decoder_generate(lin, torch, dev)

    cpu = None
    if not args.no_cpu and not args.quick and rank == 0:
        log("CPU baseline")
        cpu = cpu_baseline()

    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_step * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "batch-1 decode projection set of one Qwen3-VL-2B text layer + lm_head, "
                               "W8A32: QKV 4096x2048, O 2048x2048, gate_up 12288x2048, down 2048x6144, "
                               "lm_head 151936x2048; the timed steps in one HIP graph, step i on layer "
                               "copy i % 28 of 28 distinct ones (every step's weights from HBM)",
                   "step_bytes": step_bytes, "launches_per_step": len(LAYER_SHAPES) + 1},
        "wall_s": round(wall, 3),
        "roofline": roofline,
        "graph_per_step": graph_per_step,
        "decode_step_28_layers": step28,
        "lm_head_greedy": greedy,
        "gemv_6144x2048": single,
        "decoder_greedy": dec,
        "w8a8_prefill": prefill,
        "w8a32_decode_rows": rows,
        "w8a32_reference_rows": ref_rows,
        "w8a16_sweep": sweep,
        "w8a32_prefill": pre32,
        "host_abi": host,
        "cpu_baseline": cpu,
    }
    if rank == 0:
        print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
