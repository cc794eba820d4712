"""bench.py's command-line contract that holds without a GPU."""

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args],
                          capture_output=True, text=True, timeout=300)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = _bench("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""


def test_traffic_figure_comes_from_the_committed_profile():
    sys.path.insert(0, ROOT)
    import bench

    assert bench.profiled_traffic() is not None
    assert bench.profiled_traffic() > bench.decode_launch_bytes(bench.workloads.cfg2_lens(0))
