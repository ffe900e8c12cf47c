"""bench.py reports the measured HBM traffic of the GEMV (roofline.traffic)
and takes the GEMV kernel time per step (roofline.frac) from committed
rocprofv3 summaries only while they were taken on the current GEMV sources:
the recorded SHA-256 of csrc/gemv.hip and csrc/tl_common.h must match the
tree, and a changed source turns the figure into null (traffic) or the
run's own HIP-event figure (frac) with the reason.  The kernel trace summary
(bench.py --summarize-trace) counts only the launches between the marker
launches that bracket each timed replay."""
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_traffic_summary_matches_the_gemv_sources():
    traffic, note = bench.measured_traffic()
    assert traffic is not None, note
    # within 5% of the algorithmic bytes per launch of the benchmark's step
    alg = sum(bench.gemv_bytes(N, K) for (_, N, K) in bench.LAYER_SHAPES + [bench.LM_HEAD]) / 5
    assert 1.0 <= traffic / alg <= 1.05


def test_changed_sources_make_the_figure_stale(tmp_path, monkeypatch):
    src = tmp_path / "gemv.hip"
    src.write_bytes(bench.GEMV_SOURCES[0].read_bytes() + b"\n// edited\n")
    monkeypatch.setattr(bench, "GEMV_SOURCES", [src, bench.GEMV_SOURCES[1]])
    traffic, note = bench.measured_traffic()
    assert traffic is None and note.startswith("stale")


def _synthetic_trace(path, steps, replays, extra_inside=False):
    """A kernel trace shaped like rocprofv3's kernel_trace.csv: warm-up GEMV
    launches, then per timed replay a marker, steps x 5 GEMV launches with
    known durations, a marker."""
    import csv
    cols = ["Kind", "Kernel_Name", "Start_Timestamp", "End_Timestamp", "Grid_Size_X"]
    grids = [131072, 65536, 196608, 65536, 2430976]
    durs_ns = [3000, 2500, 6000, 4000, 46000]
    t = 1_000_000
    rows = []

    def add(name, grid, d):
        nonlocal t
        rows.append({"Kind": "KERNEL_DISPATCH", "Kernel_Name": name, "Start_Timestamp": t,
                     "End_Timestamp": t + d, "Grid_Size_X": grid})
        t += d + 1000

    for j in range(10):                       # warm-up launches, outside the markers
        add("tl::gemv_i8_kernel<2, 4, 16, 0>(...)", grids[j % 5], 99000)
    add("tl::stream_read_kernel<4>(...)", 65536, 5000)   # a read-floor launch, not a marker
    for r in range(replays):
        add("tl::stream_read_kernel<4>(...)", 256, 800)
        for i in range(steps):
            for j in range(5):
                add("tl::gemv_i8_kernel<2, 4, 16, 0>(...)", grids[j], durs_ns[j] + 100 * r)
        if extra_inside:
            add("tl::pack_tiles_kernel(...)", 4096, 1000)
        add("tl::stream_read_kernel<4>(...)", 256, 800)
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=cols, quoting=csv.QUOTE_NONNUMERIC)
        w.writeheader()
        w.writerows(rows)
    return sum(durs_ns) / 1000.0


def test_trace_summary_counts_only_the_timed_replays(tmp_path):
    csv_path = tmp_path / "run_kernel_trace.csv"
    base_us = _synthetic_trace(csv_path, steps=4, replays=5)
    md = bench.summarize_trace(str(csv_path), 4, "rocprofv3 ... -- python3 bench.py --steps 4")
    rec = {}
    for line in md.splitlines():
        if ":" in line and line.split(":", 1)[0] in ("kernel_us_per_step", "timed_replays", "steps"):
            k, v = line.split(":", 1)
            rec[k] = v.strip()
    # replay r adds 0.1 us per launch; the median replay is r = 2
    assert abs(float(rec["kernel_us_per_step"]) - (base_us + 5 * 0.2)) < 1e-6
    assert rec["timed_replays"] == "5" and rec["steps"] == "4"
    assert "| lm_head 151936x2048 |" in md


def test_trace_summary_rejects_foreign_launches_between_markers(tmp_path):
    import pytest
    csv_path = tmp_path / "run_kernel_trace.csv"
    _synthetic_trace(csv_path, steps=2, replays=3, extra_inside=True)
    with pytest.raises(SystemExit):
        bench.summarize_trace(str(csv_path), 2, "cmd")


def test_roofline_frac_follows_the_committed_trace_only_when_current(tmp_path, monkeypatch):
    csv_path = tmp_path / "run_kernel_trace.csv"
    base_us = _synthetic_trace(csv_path, steps=3, replays=3)
    summary = tmp_path / "summary.md"
    summary.write_text(bench.summarize_trace(str(csv_path), 3, "cmd"))
    monkeypatch.setattr(bench, "TRACE_SUMMARY", summary)
    us, note = bench.profiled_step_kernel_us(3)
    assert abs(us - (base_us + 5 * 0.1)) < 1e-6, note
    us, note = bench.profiled_step_kernel_us(20)          # another step count
    assert us is None and "steps" in note
    src = tmp_path / "gemv.hip"
    src.write_bytes(bench.GEMV_SOURCES[0].read_bytes() + b"\n// edited\n")
    monkeypatch.setattr(bench, "GEMV_SOURCES", [src, bench.GEMV_SOURCES[1]])
    us, note = bench.profiled_step_kernel_us(3)
    assert us is None and "stale" in note


def test_committed_trace_summary_is_current():
    """The committed kernel trace of the benchmark's command was taken on the
    current GEMV sources at the driver's step count, so bench.py takes
    roofline.frac from it."""
    us, note = bench.profiled_step_kernel_us(20)
    assert us is not None, note
    alg = sum(bench.gemv_bytes(N, K) for (_, N, K) in bench.LAYER_SHAPES + [bench.LM_HEAD])
    assert 0.3 < alg / (us * 1e-6) / 8e12 < 1.0
