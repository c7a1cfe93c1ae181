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


def test_cpu_baseline_times_the_stock_torch_path():
    """The CPU baseline is the stock PyTorch FP32 math (the oracle's torch
    restatement), on configs 1, 3 and 4 in full."""
    sys.path.insert(0, str(ROOT))
    import bench

    doc = bench.cpu_baseline.__doc__
    assert "stock PyTorch math in FP32" in doc
    assert all(f"config {c}" in doc for c in (1, 3, 4))
    src = (ROOT / "bench.py").read_text()
    assert "from oracle.stock_torch import" in src
