"""bench.py's contract on the CPU: the figures its roofline reads from the committed
profiles, and the refusal of more than one GPU."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_rocprof_averages_of_every_decode_kernel_are_committed():
    for stage in ("decode_router_shared", "decode_experts_gate_up", "decode_down_merge"):
        us = bench.rocprof_avg_us_from_profiles(stage)
        assert us is not None and 1.0 < us < 50.0, stage
    assert bench.rocprof_avg_us_from_profiles("no_such_kernel") is None


def test_headline_fraction_recomputes_from_the_profiles():
    """The dominant kernel's fraction at the committed rocprof average: its algorithmic
    bytes (16 gate/up matrices of one 8-bit [512 x 2048] expert, x, 8 activation rows) over
    that duration, against 8 TB/s."""
    b = 16 * bench.qbytes(1, bench.I, bench.H, 8) + bench.H * 2 + 8 * bench.I * 4
    assert b == 17846272
    us = bench.rocprof_avg_us_from_profiles("decode_experts_gate_up")
    frac = b / (us * 1e3) / bench.PEAK_HBM_GBS
    assert 0.1 < frac < 1.0
    traffic = bench.traffic_from_profiles("decode_experts_gate_up")
    assert traffic is not None and 0.95 * b < traffic < 1.2 * b


@pytest.mark.parametrize("gpus", ["2", "8"])
def test_more_than_one_gpu_is_refused(gpus):
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", gpus],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
