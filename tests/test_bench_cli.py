"""CPU: bench.py's contract pieces that need no GPU -- the one-GPU refusal and the workload table."""

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 2
    assert "exactly one GPU" in r.stderr


def test_workloads_and_flop_counts():
    sys.path.insert(0, ROOT)
    import bench
    assert set(bench.WORKLOADS) >= {"c1", "c2", "c3", "c4", "c5", "c2_train", "swa_bf16", "swa_bf16_450m"}
    c3 = bench.WORKLOADS["c3"]
    assert (c3["B"], c3["H"], c3["T"], c3["D"], c3["W"]) == (4, 16, 8192, 64, 1024)
    # in-window pairs of C3: the ramp of the first W queries plus W per remaining query
    assert bench.in_window_pairs(8192, 1024) == 1024 * 1025 // 2 + (8192 - 1024) * 1024
    assert 4 * 64 * 4 * 16 * bench.in_window_pairs(8192, 1024) == 128_857_407_488
