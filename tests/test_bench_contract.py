"""bench.py's traffic figures come from the committed rocprofv3 summary: the kernel names the line
looks up must be present there (a renamed kernel would silently report null)."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_bench_traffic_kernels_are_in_the_committed_profile():
    import bench
    for name in (bench.ROOFLINE_KERNEL, bench.TOPK_KERNEL):
        t = bench.measured_traffic(name)
        assert t is not None and t > 0, name
