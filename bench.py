"""Benchmark of the INT8 linear path on one MI355X.

Workload (a "step" = one decoded token's linear layers, W8A32 batch==1):
  28 layers x {QKV 4096x2048, O 2048x2048, gate_up 12288x2048, down 2048x6144}
  + lm_head 151936x2048, every matrix distinct (1.72 GB of int8 weights, far
  beyond the 256 MB Infinity Cache), per-row fp32 scales, fp32 activations
  ~N(0,1) resident in HBM, synthetic data.
The step is captured once in a HIP graph (113 GEMV launches) and replayed.

value   = algorithmic bytes of one step / step time (GB/s); bytes per GEMV
          launch are N*K + 4N + 4K + 4N (weights, scales, x, y).
roofline: the GEMV kernel family, bytes per launch over its average launch
          duration (HIP events around each launch on the launch stream),
          against the 8 TB/s HBM peak.
Also: W8A8 prefill TOPS (M=1024; N=6144,K=2048 and N=2048,K=6144; includes
the per-token quantization kernel), and the CPU baseline (the oracle's M=1
GEMV, OpenMP on the host cores) on a bounded sample.
"""
from __future__ import annotations

import argparse
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
LAYERS = 28
LAYER_SHAPES = [("qkv", 4096, 2048), ("o", 2048, 2048), ("gate_up", 12288, 2048), ("down", 2048, 6144)]
LM_HEAD = ("lm_head", 151936, 2048)
METRIC = "INT8 GEMV HBM GB/s + decode tok/s; W8A8 prefill TOPS (Qwen3-VL-2B decoder)"


def gemv_bytes(N, K):
    return N * K + 4 * N + 4 * K + 4 * N


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def build_decode_set(lin, torch, dev, seed=0):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    items = []
    shapes = [(f"l{l}.{n}", N, K) for l in range(LAYERS) for (n, N, K) in LAYER_SHAPES] + [LM_HEAD]
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


def time_kernels(lin, torch, items, stream, reps):
    """Average duration of each GEMV launch, HIP events on the launch stream."""
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in items]
    tot = np.zeros(len(items))
    with torch.cuda.stream(stream):
        for _ in range(reps):
            for i, (_, _, _, W, x, y) in enumerate(items):
                ev[i][0].record(stream)
                lin.w8a32_linear_dev(x, W, y, stream=stream)
                ev[i][1].record(stream)
            stream.synchronize()
            for i in range(len(items)):
                tot[i] += ev[i][0].elapsed_time(ev[i][1])
    return tot / reps * 1e-3  # seconds per launch


def bench_w8a8_prefill(lin, torch, dev, reps=20):
    out = {}
    tot_ops, tot_t = 0.0, 0.0
    for (N, K) in [(6144, 2048), (2048, 6144)]:
        M = 1024
        copies = max(2, int(np.ceil(512e6 / (N * K))))      # rotate > 512 MB of weights
        Ws = []
        for c in range(copies):
            w = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev)
            s = torch.rand(N, device=dev) * 0.018 + 0.002
            Ws.append(lin.DeviceWeights.from_codes(w, s))
        x = torch.randn((M, K), device=dev)
        y = torch.empty((M, N), device=dev)
        st = torch.cuda.current_stream()
        for i in range(3):
            lin.w8a8_linear_f32_dev(x, Ws[i % copies], y, stream=st)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        for i in range(reps):
            lin.w8a8_linear_f32_dev(x, Ws[i % copies], y, stream=st)
        e1.record(st)
        torch.cuda.synchronize()
        t = e0.elapsed_time(e1) * 1e-3 / reps
        ops = 2.0 * M * N * K
        out[f"M{M}_N{N}_K{K}"] = {"us": round(t * 1e6, 2), "tops": round(ops / t / 1e12, 1),
                                   "frac_int8_peak": round(ops / t / 1e12 / INT8_PEAK_TOPS, 4)}
        tot_ops += ops
        tot_t += t
        for W in Ws:
            W.close()
    out["tops"] = round(tot_ops / tot_t / 1e12, 1)
    out["frac_int8_peak"] = round(tot_ops / tot_t / 1e12 / INT8_PEAK_TOPS, 4)
    out["includes"] = "per-token activation quantization kernel + int8 MFMA GEMM, fp32 in/out"
    return out


def cpu_baseline(seconds=12.0):
    """The oracle's M=1 GEMV (same formula as the reference's w8a32_gemv) on the
    host cores; the per-token time is 28 x the layer set + lm_head."""
    from oracle import oracle as orc
    native = True
    try:
        orc.build(native=True)
    except Exception:
        native = False
    try:
        cores = len(os.sched_getaffinity(0))
    except Exception:
        cores = os.cpu_count() or 1
    cores = max(1, min(cores, 16))
    rng = np.random.default_rng(0)
    shapes = [(n, N, K) for (n, N, K) in LAYER_SHAPES] + [LM_HEAD]
    per = {}
    budget = seconds / len(shapes)
    for (name, N, K) in shapes:
        w = rng.integers(-127, 128, (N, K), dtype=np.int8)
        s = rng.uniform(0.002, 0.02, N).astype(np.float32)
        x = rng.standard_normal(K, dtype=np.float32)
        y = np.empty(N, np.float32)
        orc.w8a32_gemv_timed(x, w, s, y, cores, native=native)   # warm-up
        times = []
        t_end = time.perf_counter() + budget
        while time.perf_counter() < t_end or len(times) < 3:
            t0 = time.perf_counter()
            orc.w8a32_gemv_timed(x, w, s, y, cores, native=native)
            times.append(time.perf_counter() - t0)
        per[name] = float(np.median(times))
    t_tok = LAYERS * sum(per[n] for (n, _, _) in LAYER_SHAPES) + per["lm_head"]
    step_bytes = LAYERS * sum(gemv_bytes(N, K) for (_, N, K) in LAYER_SHAPES) + gemv_bytes(*LM_HEAD[1:])
    return {"value": round(step_bytes / t_tok / 1e9, 2), "unit": "GB/s", "cores": cores, "kind": "port",
            "tok_s": round(1.0 / t_tok, 2),
            "sample": f"oracle M=1 GEMV ({'-march=native' if native else 'x86-64-v3'}, OpenMP) timed on "
                      f"one layer set + lm_head (median of repeats, ~{seconds:.0f}s); per-token time = "
                      f"28 x layer set + lm_head"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-prefill", action="store_true", help="skip the W8A8 prefill timing")
    ap.add_argument("--kernel-reps", type=int, default=5)
    args = ap.parse_args()
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

    log("building the decode set (1.72 GB of int8 weights)")
    items = build_decode_set(lin, torch, dev)
    step_bytes = sum(gemv_bytes(N, K) for (_, N, K, *_r) in items)
    stream = torch.cuda.Stream()

    log("warm-up (eager) and graph capture")
    with torch.cuda.stream(stream):
        for _ in range(max(1, args.warmup)):
            run_step(lin, items, stream)
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        run_step(lin, items, stream)
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()

    log(f"timing {args.steps} graph replays")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    t_step = e0.elapsed_time(e1) * 1e-3 / args.steps
    value = step_bytes / t_step / 1e9

    log("per-launch kernel timing (events)")
    kt = time_kernels(lin, torch, items, stream, args.kernel_reps)
    shapes = {}
    for (name, N, K, *_r), t in zip(items, kt):
        key = name.split(".")[-1]
        d = shapes.setdefault(key, {"N": N, "K": K, "bytes": gemv_bytes(N, K), "t": []})
        d["t"].append(t)
    per_shape = {}
    for key, d in shapes.items():
        t = float(np.mean(d["t"]))
        per_shape[key] = {"N": d["N"], "K": d["K"], "us": round(t * 1e6, 2),
                          "GBps": round(d["bytes"] / t / 1e9, 1),
                          "frac_hbm": round(d["bytes"] / t / 1e9 / HBM_PEAK_GBS, 4)}
    avg_bytes = step_bytes / len(items)
    avg_t = float(np.mean(kt))
    achieved = avg_bytes / avg_t / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                "kernel": "gemv_i8_kernel (all 113 launches of a step)",
                "bytes_per_launch": round(avg_bytes), "avg_launch_us": round(avg_t * 1e6, 2),
                "per_shape": per_shape}

    prefill = None
    if not args.no_prefill:
        log("W8A8 prefill timing")
        prefill = bench_w8a8_prefill(lin, torch, dev)

    cpu = None
    if not args.no_cpu and rank == 0:
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
        "config": {"workload": "decode projection set of the Qwen3-VL-2B text decoder, W8A32 batch=1: "
                               "28 x (QKV 4096x2048, O 2048x2048, gate_up 12288x2048, down 2048x6144) "
                               "+ lm_head 151936x2048, distinct weights, HIP-graph replay",
                   "step_bytes": step_bytes, "launches_per_step": len(items)},
        "decode_tok_s": round(1.0 / t_step, 1),
        "wall_s": round(wall, 3),
        "roofline": roofline,
        "w8a8_prefill": prefill,
        "cpu_baseline": cpu,
    }
    if rank == 0:
        print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
