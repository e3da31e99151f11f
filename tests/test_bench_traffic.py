"""bench.py's roofline.traffic comes from the committed counter summary only
while the kernel sources are the ones it was measured on (no GPU)."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402
import pytest  # noqa: E402


def test_traffic_summary_matches_the_sources():
    traffic, commit = bench.measured_traffic(16, "q4_k_m", 4096)
    if traffic is None:
        pytest.skip("the traffic summary was measured on other kernel sources (bench reports null)")
    assert commit
    # 1.0-1.1x the algorithmic bytes of a 4096-context pass (15.46 GB), per 16-pass launch
    assert 16 * 15.4e9 < traffic < 16 * 17.0e9


def test_traffic_is_null_for_other_sources_or_workloads(monkeypatch):
    assert bench.measured_traffic(16, "bf16", 4096) == (None, None)
    assert bench.measured_traffic(16, "q4_k_m", 8192) == (None, None)
    monkeypatch.setattr(bench, "kernel_source_digest", lambda: "0" * 64)
    assert bench.measured_traffic(16, "q4_k_m", 4096) == (None, None)
