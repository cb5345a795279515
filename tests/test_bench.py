"""bench.py's command line (no GPU): one GPU only, and the default step
counts (500 timed after 50 warm-up steps for the microsecond configs 1-2,
50 after 10 for the others)."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU only" in (r.stdout + r.stderr)


@pytest.mark.parametrize("argv, steps, warmup", [
    ([], 500, 50),
    (["--config", "1"], 500, 50),
    (["--config", "3"], 50, 10),
    (["--config", "5"], 50, 10),
    (["--config", "2", "--steps", "7", "--warmup", "2"], 7, 2),
])
def test_default_steps(monkeypatch, argv, steps, warmup):
    import bench

    monkeypatch.setattr(sys, "argv", ["bench.py", *argv])
    args = bench.parse()
    assert (args.steps, args.warmup) == (steps, warmup)
    assert args.gpus == 1
