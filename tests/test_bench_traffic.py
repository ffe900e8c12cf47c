"""bench.py reports the measured HBM traffic of the GEMV (roofline.traffic)
from the committed rocprofv3 summary only while that summary was taken on the
current GEMV sources: the recorded SHA-256 of csrc/gemv.hip and
csrc/tl_common.h must match the tree, and a changed source turns the figure
into null with the reason."""
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
