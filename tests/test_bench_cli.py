"""bench.py contract checks that need no GPU."""

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_multi_gpu_request_exits_with_message():
    res = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True,
                         text=True, timeout=120)
    assert res.returncode == 2
    assert "one MI355X" in res.stderr


def test_cpu_baseline_sample_runs_quickly(monkeypatch):
    sys.path.insert(0, str(ROOT))
    import bench

    monkeypatch.setattr(bench, "O", 384)
    # The oracle leg is the checker, timed on host cores; keep its contract.
    line = bench.cpu_baseline.__doc__
    assert "numpy oracle" in line
