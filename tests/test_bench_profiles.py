"""The bench line's `roofline.traffic` comes from the committed rocprofv3 counter summaries:
every configuration the default run reports has one, and each parses to a traffic figure at
least as large as the algorithmic bytes it states (no GPU needed)."""
import re
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402

WORKLOADS = ["hunyuan_480p"] + [w[0] for w in bench.OTHER_WORKLOADS] + [bench.SEQUENCE_WORKLOAD[0]]


@pytest.mark.parametrize("workload", WORKLOADS)
def test_every_reported_configuration_has_counted_traffic(workload):
    traffic = bench.measured_traffic(workload)
    assert traffic is not None, f"profiles/sparse_attention_{workload}_traffic.txt missing or without a figure"
    text = (ROOT / "profiles" / f"sparse_attention_{workload}_traffic.txt").read_text()
    # Every summary names the commands that made it and the two counters it was derived from.
    assert "rocprofv3 --pmc FETCH_SIZE" in text and "rocprofv3 --pmc WRITE_SIZE" in text
    m = re.search(r"^algorithmic_bytes_per_launch:\s*([0-9.eE+]+)", text, re.M)
    if m:
        assert traffic >= float(m.group(1))


def test_traffic_is_fetch_plus_write_scaled_by_the_copy_calibration():
    """traffic = FETCH_SIZE x 2 + WRITE_SIZE x 1 (KiB per dispatch), the factors a plain device
    copy of known size gives, wherever a summary lists the two counters."""
    for workload in WORKLOADS:
        text = (ROOT / "profiles" / f"sparse_attention_{workload}_traffic.txt").read_text()
        fetch = re.search(r"^FETCH_SIZE_KiB_per_dispatch:\s*([0-9.eE+]+)", text, re.M)
        write = re.search(r"^WRITE_SIZE_KiB_per_dispatch:\s*([0-9.eE+]+)", text, re.M)
        if not (fetch and write):
            continue
        expected = (2.0 * float(fetch.group(1)) + float(write.group(1))) * 1024
        assert bench.measured_traffic(workload) == pytest.approx(expected, rel=2e-3), workload
