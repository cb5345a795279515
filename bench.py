#!/usr/bin/env python3
"""Benchmark of the SWTCF / spmm_cnic hot path on one MI355X.

Default workload ("config 2"): R-MAT graph, 169k
nodes, 1.17M nnz, sym-normalised fp32 values, X = N(0,1) [169k x 128]; one
step = one forward BCSR SpMM (Y = A X) over the whole graph, inputs resident
in HBM.  --config 1/3 select the other single-GPU SpMM configurations.

Prints one JSON line with GFLOP/s (2*nnz*F per step), the HBM roofline of the
kernel (algorithmic bytes 4F(n_src+n_dst) + 8 nnz + 4(n_dst+1) per launch
over the HIP-event-timed launch duration) and the CPU baseline (the oracle's
CSR SpMM on the host cores, the same matrix, checked against the GPU result).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "SpMM GFLOP/s (2·nnz·F) + % HBM roofline; GCN layer fwd+bwd ms at 1 GPU"
HBM_PEAK_GBPS = 8000.0
FP32_PEAK_TFLOPS = 157.3

WORKLOADS = {
    1: "config1: uniform 4096 nodes x 16 nnz/row, F=32, SWTCF convert + SWTCF SpMM",
    2: "config2: R-MAT (0.57,0.19,0.19) 169k nodes, 1.17M nnz, sym-normalised, F=128, forward BCSR SpMM",
    3: "config3: R-MAT (0.57,0.19,0.19) 233k nodes, 114M nnz, sym-normalised, F=602, forward BCSR SpMM",
}


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--config", type=int, default=2, choices=sorted(WORKLOADS))
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-threads", type=int, default=0, help="0 = all host cores")
    p.add_argument("--copy-calibration-mib", type=int, default=0,
                   help="first run one plain device copy of this many MiB (scale for rocprofv3 FETCH/WRITE_SIZE)")
    return p.parse_args()


def bytes_alg(n_src, n_dst, nnz, F):
    return 4.0 * F * (n_src + n_dst) + 8.0 * nnz + 4.0 * (n_dst + 1)


def cpu_baseline(rows, cols, vals, X, n, threads, Y_gpu, max_nnz):
    """The oracle's CSR SpMM (OpenMP, fp64 accumulation of TF32-rounded
    inputs) on the host cores over the leading rows holding at most max_nnz
    nonzeros (the whole matrix when it is smaller): median of 5 after 1
    warm-up.  Also the parity check of the GPU result on those rows (rel-L2).
    Returns (seconds, threads, rel_l2, rows, nnz) of the sample."""
    import numpy as np

    import oracle
    from tcc_amd.graphs import to_csr_numpy

    threads = threads or os.cpu_count() or 1
    rowptr, colind, v = to_csr_numpy(rows, cols, n, vals)
    R = int(np.searchsorted(rowptr, max_nnz, side="right")) - 1
    R = max(1, min(n, R))
    nz = int(rowptr[R])
    rp = np.ascontiguousarray(rowptr[: R + 1])
    ci = np.ascontiguousarray(colind[:nz])
    vv = None if v is None else np.ascontiguousarray(v[:nz])
    Xc = X.cpu().numpy()
    oracle.csr_spmm(rp, ci, vv, Xc, use_tf32=True, threads=threads)
    ts = []
    Y = None
    for _ in range(5):
        t0 = time.perf_counter()
        Y = oracle.csr_spmm(rp, ci, vv, Xc, use_tf32=True, threads=threads)
        ts.append(time.perf_counter() - t0)
    t = sorted(ts)[len(ts) // 2]
    yg = Y_gpu[:R].cpu().numpy().astype(np.float64)
    rel = float(np.linalg.norm(yg - Y) / max(np.linalg.norm(Y), 1e-30))
    return t, threads, rel, R, nz


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no multi-GPU path",
              file=sys.stderr)
        return 2
    import torch

    from tcc_amd import swtcf
    from tcc_amd.graphs import CONFIGS, make_features, make_graph

    assert torch.cuda.is_available(), "bench.py needs the GPU"
    torch.cuda.set_device(0)
    cfg = CONFIGS[args.config]
    n, F = cfg["n"], cfg["F"]
    t0 = time.time()
    rows, cols, vals = make_graph(args.config, device="cuda")
    nnz = rows.numel()
    print(f"[bench] config {args.config}: n={n} nnz={nnz} F={F} generated in {time.time() - t0:.1f}s",
          file=sys.stderr, flush=True)
    X = make_features(n, F, cfg["seed"], dist="uniform" if args.config == 1 else "normal", device="cuda")
    r32 = rows.to(torch.int32).contiguous()
    c32 = cols.to(torch.int32).contiguous()
    stream = torch.cuda.current_stream()

    extra = {}
    if args.config == 1:
        m = swtcf.DeviceSWTCFMatrix(n, n, nnz, 16)
        ws = swtcf.SWTCFConvertWorkspace(nnz, n, 16)
        swtcf.convertCOOToSWTCF(r32, c32, nnz, m, ws)
        torch.cuda.synchronize()
        c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        c0.record(stream)
        for _ in range(20):
            swtcf.convertCOOToSWTCF(r32, c32, nnz, m, ws)
        c1.record(stream)
        torch.cuda.synchronize()
        conv_ms = c0.elapsed_time(c1) / 20
        assert ws.device_error() == 0
        extra["convert_ms"] = round(conv_ms, 4)
        extra["convert_gedges_per_s"] = round(nnz / conv_ms / 1e6, 3)
        Y = torch.zeros((n, F), device="cuda")

        def step():
            swtcf.swtcf_spmm(m, X, Y, 12)

        kernel = "swtcf_spmm_kernel"
    else:
        A = swtcf.coo_to_bcsr(r32, c32, vals, n, n)
        Y = torch.empty((A.view.num_rowWindows * 8, F), device="cuda")
        extra["blocks"] = A.view.num_TCBlocks

        def step():
            swtcf.bcsr_spmm(A, X, Y)

        kernel = "gather_kernel"

    if args.copy_calibration_mib:
        nfl = args.copy_calibration_mib * (1 << 20) // 4
        a_src = torch.ones(nfl, device="cuda")
        a_dst = torch.empty_like(a_src)
        torch.cuda.synchronize()
        a_dst.copy_(a_src)  # reads and writes exactly copy_calibration_mib MiB
        torch.cuda.synchronize()
        del a_src, a_dst

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    flops = 2.0 * nnz * F
    gflops = flops / (ms * 1e-3) / 1e9
    b_alg = bytes_alg(n, n, nnz, F)
    achieved = b_alg / (ms * 1e-3) / 1e9
    traffic = None
    tf = os.path.join(ROOT, "profiles", f"traffic_config{args.config}.json")
    if os.path.exists(tf):
        with open(tf) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    if args.config == 1:
        torch.cuda.synchronize()
        Y.zero_()
        step()
    torch.cuda.synchronize()

    cpu = None
    if not args.no_cpu_baseline:
        t_cpu, threads, rel, R, nz = cpu_baseline(rows, cols, vals, X, n, args.cpu_threads, Y, 16_000_000)
        whole = nz == nnz
        what = (f"whole config-{args.config} matrix ({nnz} nnz, F={F})" if whole else
                f"rows 0..{R - 1} of config {args.config} ({nz} of {nnz} nnz, F={F})")
        cpu = {"value": round(2.0 * nz * F / t_cpu / 1e9, 3), "unit": "GFLOP/s", "cores": threads, "kind": "port",
               "sample": f"{what}; oracle CSR SpMM, fp64 accumulation of TF32-rounded inputs, OpenMP over rows, "
                         f"median of 5 after 1 warm-up",
               "ms": round(t_cpu * 1e3, 3)}
        extra["parity_rel_l2_vs_cpu"] = rel
        extra["parity_rows"] = R

    line = {
        "metric": METRIC,
        "value": round(gflops, 3),
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded generator, see tcc_amd/graphs.py)",
        "config": {"workload": WORKLOADS[args.config], "n": n, "nnz": nnz, "F": F},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic, "kernel": kernel,
                     "bytes_alg_per_launch": b_alg},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
