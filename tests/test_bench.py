"""bench.py's command line and roofline arithmetic (no GPU): one GPU only,
the default configuration (config 3) and step counts (500 timed after 50
warm-up steps for the microsecond configs 1-2, 50 after 10 for the others),
and the roofline min(157.3 TFLOP/s, AI x 8 TB/s)."""
import json
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


@pytest.mark.parametrize("argv, config, steps, warmup", [
    ([], 3, 50, 10),
    (["--config", "1"], 1, 500, 50),
    (["--config", "2"], 2, 500, 50),
    (["--config", "5"], 5, 50, 10),
    (["--config", "2", "--steps", "7", "--warmup", "2"], 2, 7, 2),
])
def test_default_steps(argv, config, steps, warmup):
    import bench

    args = bench.parse(argv)
    assert (args.config, args.steps, args.warmup) == (config, steps, warmup)
    assert args.gpus == 1


def test_roofline_config3_is_fp32_bound():
    """Config 3 (233k nodes, 114M nnz, F=602): AI = 67.5 FLOP/B, so the fp32
    roof (157.3 TFLOP/s) binds before AI x 8 TB/s = 540 TFLOP/s."""
    import bench

    n, nnz, F = 233_000, 114_000_000, 602
    flops = 2.0 * nnz * F
    b = bench.bytes_alg(n, n, nnz, F)
    assert b == 4.0 * F * 2 * n + 8.0 * nnz + 4.0 * (n + 1)
    ms = 10.0
    r = bench.roofline(flops, b, ms, None, "k")
    assert r["bound"] == "mfma" and r["unit"] == "TFLOP/s" and r["peak"] == 157.3
    assert abs(r["arith_intensity"] - flops / b) < 1e-3
    assert abs(r["achieved"] - flops / 1e-2 / 1e12) < 1e-3
    # frac = (flops / t) / min(157.3 TF, AI * 8 TB/s)
    assert abs(r["frac"] - (flops / 1e-2) / min(157.3e12, flops / b * 8e12)) < 1e-4
    assert r["traffic"] is None and "l2_fabric_traffic" not in r
    assert abs(r["hbm_fraction_alg"] - b / 1e-2 / 8e12) < 1e-4


def test_roofline_config2_is_hbm_bound():
    import bench

    n, nnz, F = 169_000, 1_170_000, 128
    flops = 2.0 * nnz * F
    b = bench.bytes_alg(n, n, nnz, F)
    r = bench.roofline(flops, b, 0.08, {"hbm_bytes_per_launch": 4e8, "file": "x"}, "k")
    assert r["bound"] == "hbm" and r["unit"] == "GB/s" and r["peak"] == 8000.0
    assert abs(r["achieved"] - b / 0.08e-3 / 1e9) < 1e-2
    assert abs(r["frac"] - (flops / 0.08e-3) / min(157.3e12, flops / b * 8e12)) < 1e-4
    assert r["traffic"] == 4e8
    assert abs(r["l2_fabric_traffic"]["GBps"] - 4e8 / 0.08e-3 / 1e9) < 0.1
    assert abs(r["hbm_fraction_alg"] - b / 0.08e-3 / 8e12) < 1e-4


def test_traffic_files_name_their_sources():
    """A counter-measured traffic figure is only used while the kernel
    sources it was measured on are unchanged."""
    import bench

    pdir = os.path.join(ROOT, "profiles")
    for name in sorted(os.listdir(pdir)):
        if not (name.startswith("traffic_config") and name.endswith(".json")):
            continue
        with open(os.path.join(pdir, name)) as f:
            d = json.load(f)
        cfg = int(name[len("traffic_config"):-len(".json")])
        t = bench.traffic_of(cfg)
        if "sources" in d:
            for p in d["sources"]:
                assert os.path.exists(os.path.join(ROOT, p)), p
        if t is not None:
            assert t["hbm_bytes_per_launch"] == d["hbm_bytes_per_launch"]
