"""bench.py's JSON line on the GPU: a short config-2 run in a child process,
every field the driver reads, and the roofline arithmetic."""
import json
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_line_config2():
    r = subprocess.run([sys.executable, "-u", os.path.join(ROOT, "bench.py"), "--config", "2", "--steps", "5",
                        "--warmup", "1", "--no-cpu-baseline"], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [l for l in r.stdout.splitlines() if l.startswith("{")]
    assert len(lines) == 1, r.stdout[-2000:]
    d = json.loads(lines[0])
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
              "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert k in d, k
    assert d["n_gpus"] == 1 and d["steps"] == 5 and d["warmup"] == 1
    assert d["unit"] == "GFLOP/s" and d["higher_is_better"] is True and d["vs_baseline"] is None
    assert d["value"] > 0 and d["ms_per_step"] > 0
    # the median of the per-step event times, beside the mean
    assert 0 < d["median_ms_per_step"] <= 2 * d["ms_per_step"]
    # GFLOP/s = 2 nnz F / step time
    c = d["config"]
    assert "workload" in c and c["F"] == 128
    assert abs(d["value"] - 2.0 * c["nnz"] * c["F"] / (d["ms_per_step"] * 1e-3) / 1e9) <= 1e-3 * d["value"] + 1e-3
    roof = d["roofline"]
    for k in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert k in roof, k
    assert roof["bound"] == "hbm" and roof["unit"] == "GB/s" and roof["peak"] == 8000.0
    assert abs(roof["frac"] - roof["achieved"] / roof["peak"]) < 1e-3
    assert d["cpu_baseline"] is None  # --no-cpu-baseline
