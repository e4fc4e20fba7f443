"""The committed rocprofv3 summaries that bench.py reads its roofline `traffic` from: every workload with a traffic
profile has one, every kernel the summary lists was dispatched in the counter runs, and the calibrated traffic is
positive and not below the algorithmic bytes by more than cache noise (the workloads rotate over >= 1 GiB of copies,
so no cache can serve a read-once stream)."""
import os
import re

import pytest

import bench

PROFILES = os.path.join(bench.ROOT, "profiles")
WITH_TRAFFIC = sorted(n for n, c in bench.WORKLOADS.items() if c.traffic_profile)


def _fields(path):
    with open(path, encoding="utf-8") as f:
        text = f.read()
    alg = re.search(r"^algorithmic bytes per launch \(bench.py\): (\d+)$", text, re.M)
    traffic = re.search(r"^traffic_bytes_per_launch: (\d+)$", text, re.M)
    return text, int(alg.group(1)) if alg else None, int(traffic.group(1)) if traffic else None


@pytest.mark.parametrize("name", WITH_TRAFFIC)
def test_traffic_summary_is_complete(name):
    cls = bench.WORKLOADS[name]
    text, alg, traffic = _fields(os.path.join(PROFILES, cls.traffic_profile))
    assert "(not dispatched)" not in text, f"{cls.traffic_profile} names a kernel the counter runs did not dispatch"
    assert "rocprofv3 --pmc FETCH_SIZE" in text and "rocprofv3 --pmc WRITE_SIZE" in text
    assert alg and traffic and traffic >= 0.95 * alg
    assert bench.read_traffic(cls) == traffic


@pytest.mark.parametrize("name", WITH_TRAFFIC)
def test_trace_summary_beside_it(name):
    trace = bench.WORKLOADS[name].traffic_profile.replace("_pmc.txt", "_trace.txt")
    with open(os.path.join(PROFILES, trace), encoding="utf-8") as f:
        text = f.read()
    assert "rocprofv3 --kernel-trace --stats" in text and f"--workload {name} " in text
