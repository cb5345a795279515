"""The command-line drivers swtcf_convert_run / swtcf_spmm_run (tcc_amd/cli,
the reference's src/swtcf_convert_main.cu and src/swtcf_spmm_main.cu over
this library): arguments, raw u32 COO inputs, printed checks and exit codes
(0 pass, 1 usage, 2 converter device error, 3 check failed, 4 I/O error)."""
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tcc_amd", "bin")
CONVERT = os.path.join(BIN, "swtcf_convert_run")
SPMM = os.path.join(BIN, "swtcf_spmm_run")


def run(cmd, timeout=120):
    return subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)


def write_coo(tmp_path, dst, src, tag="g"):
    d, s = tmp_path / f"{tag}_dst_local.bin", tmp_path / f"{tag}_src_local.bin"
    np.asarray(dst, np.uint32).tofile(d)
    np.asarray(src, np.uint32).tofile(s)
    return str(d), str(s)


def test_usage_and_io_errors(tmp_path):
    for exe in (CONVERT, SPMM):
        assert os.path.exists(exe), "build with python -m tcc_amd.build"
        r = run([exe])
        assert r.returncode == 1 and "usage" in r.stderr
        r = run([exe, str(tmp_path / "missing_dst.bin"), str(tmp_path / "missing_src.bin")])
        assert r.returncode == 4 and "cannot open" in r.stderr
    bad = tmp_path / "odd.bin"
    bad.write_bytes(b"\x01\x02\x03")
    r = run([CONVERT, str(bad), str(bad)])
    assert r.returncode == 4 and "invalid binary size" in r.stderr


def uniform(n, deg, seed):
    rng = np.random.default_rng(seed)
    keys = np.unique(np.concatenate([r * n + rng.choice(n, deg, replace=False) for r in range(n)]))
    return (keys // n).astype(np.uint32), (keys % n).astype(np.uint32)


@pytest.mark.gpu
@pytest.mark.parametrize("S", [16, 3, 32])
def test_convert_run_passes(gpu, tmp_path, S):
    from tcc_amd.graphs import rmat_graph

    rows, cols = rmat_graph(3000, 40_000, 7)
    d, s = write_coo(tmp_path, rows.numpy(), cols.numpy())
    r = run([CONVERT, d, s, str(S), "3"])
    assert r.returncode == 0, r.stdout + r.stderr
    assert "SWTCF validation: PASS" in r.stdout and "repeat-cache validation: PASS" in r.stdout
    assert "edges: 40000" in r.stdout and "GEdges/s" in r.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("tc", [12, 65])
def test_spmm_run_passes(gpu, tmp_path, tc):
    dst, src = uniform(4096, 16, 1)
    d, s = write_coo(tmp_path, dst, src)
    r = run([SPMM, d, s, str(tc), "3"])
    assert r.returncode == 0, r.stdout + r.stderr
    assert "SpMM validation: PASS" in r.stdout and "failed elements: 0 /" in r.stdout


@pytest.mark.gpu
def test_duplicate_edges_report_device_error(gpu, tmp_path):
    """A (window, dst) group with more than 8 edges (duplicates) is device
    error 1, as the reference's converter reports it (swtcf_convert.cu:186-196)."""
    dst = np.zeros(9, np.uint32)
    src = np.array([0, 1, 2, 3, 4, 5, 6, 7, 7], np.uint32)
    d, s = write_coo(tmp_path, dst, src)
    r = run([CONVERT, d, s])
    assert r.returncode == 2 and "converter device error: 1" in r.stderr
