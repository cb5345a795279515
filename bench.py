#!/usr/bin/env python3
"""Benchmark of the SWTCF / spmm_cnic hot path on one MI355X.

Default workload ("config 2"): R-MAT graph, 169k
nodes, 1.17M nnz, sym-normalised fp32 values, X = N(0,1) [169k x 128]; one
step = one forward BCSR SpMM (Y = A X) over the whole graph, inputs resident
in HBM.  The other configurations:
  --config 1  uniform 4096 x 16/row, F=32: SWTCF convert + SWTCF SpMM
  --config 3  R-MAT 233k nodes, 114M nnz, F=602: BCSR SpMM
  --config 4  R-MAT 2.45M nodes, 61.9M nnz, F=100, top-20% rows hot in HBM,
              the rest zero-copy from pinned host memory: mixed SpMM
              (BCSR over hot sources + BCSC over cold sources)
  --config 5  2-layer GCN (100 -> 256 -> 2, ReLU) on the config-4 graph: one
              full-graph training epoch (forward, loss, backward, Adam)

Prints one JSON line.  SpMM configurations report GFLOP/s (2*nnz*F per
step), the HBM roofline of the dominant kernel (algorithmic bytes
4F(n_src+n_dst) + 8 nnz + 4(n_dst+1) per launch over the HIP-event-timed
step) and the CPU baseline (the oracle's CSR SpMM on the host cores over a
bounded sample of the same matrix, also the parity check).  Config 5
reports the epoch time in ms and each layer's forward+backward time.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
import warnings

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "SpMM GFLOP/s (2·nnz·F) + % HBM roofline; GCN layer fwd+bwd ms at 1 GPU"
HBM_PEAK_GBPS = 8000.0
PCIE_PEAK_GBPS = 64.0  # PCIe Gen5 x16, one direction
# Gathers per feature row from which packing X to TF32 first pays off
# (measured: 441 -> 12% faster at config 3; 7.3 -> 23% slower at config 2).
PACK_MIN_REUSE = 16.0
# Mean blocks per row window from which the phased BCSR (column phases
# stacked, every window added with atomics) pays off, and its phase count
# (measured: config 3, 441 blocks per window, 20.0 -> 17.5 ms with 4 phases
# and 2-8 phases within 0.3 ms; config 2, 7.3 blocks per window, 78 -> 154 us
# with 2).
PHASE_MIN_BLOCKS_PER_WINDOW = 64.0
PHASES = 4

WORKLOADS = {
    1: "config1: uniform 4096 nodes x 16 nnz/row, F=32, SWTCF convert + SWTCF SpMM",
    2: "config2: R-MAT (0.57,0.19,0.19) 169k nodes, 1.17M nnz, sym-normalised, F=128, forward BCSR SpMM",
    3: "config3: R-MAT (0.57,0.19,0.19) 233k nodes, 114M nnz, sym-normalised, F=602, forward BCSR SpMM",
    4: "config4: R-MAT 2.45M nodes, 61.9M nnz, F=100, top-20% rows hot in HBM, rest pinned host: mixed SpMM",
    5: "config5: 2-layer GCN 100->256->2 (ReLU, dropout 0, Adam 0.003) on the config-4 graph, full-graph epoch",
}


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=None,
                   help="timed steps (default: 500 for the microsecond configs 1-2, else 50)")
    p.add_argument("--warmup", type=int, default=None, help="untimed steps (default: 50 for configs 1-2, else 10)")
    p.add_argument("--config", type=int, default=2, choices=sorted(WORKLOADS))
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-threads", type=int, default=0, help="0 = all host cores")
    p.add_argument("--copy-calibration-mib", type=int, default=0,
                   help="first run one plain device copy of this many MiB (scale for rocprofv3 FETCH/WRITE_SIZE)")
    args = p.parse_args()
    # A config-2 step is ~80 us: 500 of them time 40 ms of steady-state work
    # (50 took 4 ms, short enough for the clock ramp to show).
    short = args.config in (1, 2)
    if args.steps is None:
        args.steps = 500 if short else 50
    if args.warmup is None:
        args.warmup = 50 if short else 10
    return args


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


def torch_sparse_cpu(rows, cols, vals, X, n, threads, max_nnz):
    """The reference's own SpMM call, torch.sparse.mm (train/tcgnn_conv_release.py:152),
    on the host cores in fp32 with a CSR tensor, over the same leading-rows
    sample as cpu_baseline: median of 5 after 1 warm-up."""
    import numpy as np
    import torch

    from tcc_amd.graphs import to_csr_numpy

    threads = threads or os.cpu_count() or 1
    rowptr, colind, v = to_csr_numpy(rows, cols, n, vals)
    R = max(1, min(n, int(np.searchsorted(rowptr, max_nnz, side="right")) - 1))
    nz = int(rowptr[R])
    vv = np.ones(nz, np.float32) if v is None else np.asarray(v[:nz], np.float32)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")  # "sparse CSR support is in beta"
        A = torch.sparse_csr_tensor(torch.from_numpy(rowptr[: R + 1].astype(np.int64)),
                                    torch.from_numpy(colind[:nz].astype(np.int64)), torch.from_numpy(vv), size=(R, n))
    Xc = X.cpu()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        torch.sparse.mm(A, Xc)
        ts = []
        for _ in range(5):
            t0 = time.perf_counter()
            torch.sparse.mm(A, Xc)
            ts.append(time.perf_counter() - t0)
    finally:
        torch.set_num_threads(prev)
    t = sorted(ts)[len(ts) // 2]
    return {"value": round(2.0 * nz * X.shape[1] / t / 1e9, 3), "unit": "GFLOP/s", "cores": threads,
            "ms": round(t * 1e3, 3), "nnz": nz,
            "what": "torch.sparse.mm (CSR, fp32) on the host cores, the reference's own SpMM call, same sample"}


def timed(step, steps, warmup):
    """Mean ms per step over `steps` after `warmup`, timed with HIP events on
    the current stream (every launch of the step goes to that stream)."""
    import torch

    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def copy_calibration(mib):
    import torch

    nfl = mib * (1 << 20) // 4
    a_src = torch.ones(nfl, device="cuda")
    a_dst = torch.empty_like(a_src)
    torch.cuda.synchronize()
    a_dst.copy_(a_src)  # reads and writes exactly `mib` MiB
    torch.cuda.synchronize()
    del a_src, a_dst


def traffic_of(config):
    tf = os.path.join(ROOT, "profiles", f"traffic_config{config}.json")
    if os.path.exists(tf):
        with open(tf) as f:
            return json.load(f).get("hbm_bytes_per_launch")
    return None


def line_for(args, value, unit, ms, dtype, config, roofline, cpu, extra, higher=True):
    return {
        "metric": METRIC, "value": value, "unit": unit, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 5), "higher_is_better": higher, "scaling": "weak", "vs_baseline": None,
        "dtype": dtype, "data": "synthetic (seeded generator, see tcc_amd/graphs.py)", "config": config,
        "roofline": roofline, "cpu_baseline": cpu, "extra": extra,
    }


def cpu_entry(t_cpu, threads, nz, nnz, R, F, config):
    what = (f"whole config-{config} matrix ({nnz} nnz, F={F})" if nz == nnz else
            f"rows 0..{R - 1} of config {config} ({nz} of {nnz} nnz, F={F})")
    return {"value": round(2.0 * nz * F / t_cpu / 1e9, 3), "unit": "GFLOP/s", "cores": threads, "kind": "port",
            "sample": f"{what}; oracle CSR SpMM, fp64 accumulation of TF32-rounded inputs, OpenMP over rows, "
                      f"median of 5 after 1 warm-up",
            "ms": round(t_cpu * 1e3, 3)}


def swtcf_timings(torch, swtcf, m, X, n, nnz, F):
    """The SWTCF SpMM of the config-2 graph at the reference's F = 128, S = 16
    contract: fp32 X (launchSWTCFSpMM) and int8 X with per-row scales
    (launchSWTCFSpMMQuantized, src/swtcf_spmm.cu:469-502).  Y += A X is
    launched without zeroing Y between launches, as the reference times it
    (swtcf_spmm_main.cu:203-247 sets Y once)."""
    Y = torch.zeros((n, F), device="cuda")
    fp32_ms = timed(lambda: swtcf.launchSWTCFSpMM(m, X, Y), 20, 3)
    scale = X.abs().amax(dim=1).clamp_min(1e-30) / 127.0
    q = torch.round(X / scale[:, None]).clamp(-127, 127).to(torch.int8).contiguous()
    src_global = torch.arange(n, dtype=torch.int32, device="cuda")
    q_ms = timed(lambda: swtcf.launchSWTCFSpMMQuantized(m, q, scale.contiguous(), src_global, Y), 20, 3)
    gf = lambda ms: round(2.0 * nnz * F / (ms * 1e-3) / 1e9, 3)
    return {"F": F, "S": 16, "fp32_ms": round(fp32_ms, 4), "fp32_gflops": gf(fp32_ms),
            "int8_ms": round(q_ms, 4), "int8_gflops": gf(q_ms),
            "X_bytes_fp32": 4 * n * F, "X_bytes_int8": n * F + 4 * n}


def bench_spmm(args, torch, swtcf, cfg):
    """Configs 1-3: one SpMM per step."""
    from tcc_amd.graphs import make_features, make_graph

    n, F = cfg["n"], cfg["F"]
    t0 = time.time()
    rows, cols, vals = make_graph(args.config, device="cuda")
    nnz = rows.numel()
    print(f"[bench] config {args.config}: n={n} nnz={nnz} F={F} generated in {time.time() - t0:.1f}s",
          file=sys.stderr, flush=True)
    X = make_features(n, F, cfg["seed"], dist="uniform" if args.config == 1 else "normal", device="cuda")
    r32 = rows.to(torch.int32).contiguous()
    c32 = cols.to(torch.int32).contiguous()
    extra = {}
    if args.config == 1:
        m = swtcf.DeviceSWTCFMatrix(n, n, nnz, 16)
        ws = swtcf.SWTCFConvertWorkspace(nnz, n, 16)
        swtcf.convertCOOToSWTCF(r32, c32, nnz, m, ws)
        conv_ms = timed(lambda: swtcf.convertCOOToSWTCF(r32, c32, nnz, m, ws), 20, 2)
        assert ws.device_error() == 0
        extra["convert_ms"] = round(conv_ms, 4)
        extra["convert_gedges_per_s"] = round(nnz / conv_ms / 1e6, 3)
        Y = torch.zeros((n, F), device="cuda")

        def step():
            swtcf.swtcf_spmm(m, X, Y, 12)

        kernel = "swtcf_spmm_kernel"
    else:
        swtcf.coo_to_bcsr(r32, c32, vals, n, n).release()  # warm-up
        torch.cuda.synchronize()
        t_b = time.perf_counter()
        A = swtcf.coo_to_bcsr(r32, c32, vals, n, n)
        torch.cuda.synchronize()
        extra["bcsr_build_ms"] = round((time.perf_counter() - t_b) * 1e3, 3)
        extra["blocks"] = A.view.num_TCBlocks
        reuse = 8.0 * A.view.num_TCBlocks / n  # feature-row gathers per row
        extra["row_reuse"] = round(reuse, 2)
        per_window = A.view.num_TCBlocks / max(1, A.view.num_rowWindows)
        extra["blocks_per_window"] = round(per_window, 1)
        if per_window >= PHASE_MIN_BLOCKS_PER_WINDOW:
            # long windows: the phased BCSR of the same COO, built once
            t_p = time.perf_counter()
            Ap = swtcf.coo_to_bcsr(r32, c32, vals, n, n, phases=PHASES)
            torch.cuda.synchronize()
            extra["phased_build_ms"] = round((time.perf_counter() - t_p) * 1e3, 3)
            extra["phases"] = PHASES
            A.release()
            A = Ap
        Y = torch.empty((A.out_windows * 8, F), device="cuda")
        phased = f" over the {A.phases}-phase BCSR (Y zero-filled first)" if A.phases > 1 else ""
        if reuse >= PACK_MIN_REUSE:
            # each step packs X to TF32 rows of 2.5 B/element, then gathers them
            buf = torch.empty(swtcf._lib.lib().tcc_tf32_packed_bytes(n, F) + 16, dtype=torch.uint8, device="cuda")

            def step():
                swtcf.bcsr_spmm_packed(A, swtcf.tf32_pack(X, out=buf), F, Y)

            kernel = ("gather_kernel<Packed> (full chunks, then a last chunk of <= 128 features as its own launch; "
                      f"after tf32_pack_kernel, all timed){phased}")
            extra["path"] = "tf32_pack + packed gather" + phased
        else:
            def step():
                swtcf.bcsr_spmm(A, X, Y)

            kernel = "gather_kernel" + phased
            extra["path"] = "fp32 gather" + phased
    if args.config in (2, 3):
        # SWTCF conversion of the same COO (S = 16), GEdges/s as the
        # reference's converter driver prints it (swtcf_convert_main.cu:417)
        m = swtcf.DeviceSWTCFMatrix(n, n, nnz, 16)
        ws = swtcf.SWTCFConvertWorkspace(nnz, n, 16)
        conv_ms = timed(lambda: swtcf.convertCOOToSWTCF(r32, c32, nnz, m, ws), 5 if args.config == 2 else 3, 1)
        assert ws.device_error() == 0
        extra["convert_ms"] = round(conv_ms, 4)
        extra["convert_gedges_per_s"] = round(nnz / conv_ms / 1e6, 3)
        if args.config == 2:
            extra["swtcf"] = swtcf_timings(torch, swtcf, m, X, n, nnz, F)
        del m, ws
    if args.copy_calibration_mib:
        copy_calibration(args.copy_calibration_mib)
    ms = timed(step, args.steps, args.warmup)
    flops = 2.0 * nnz * F
    b_alg = bytes_alg(n, n, nnz, F)
    achieved = b_alg / (ms * 1e-3) / 1e9
    if args.config == 1:
        torch.cuda.synchronize()
        Y.zero_()
        step()
    torch.cuda.synchronize()
    cpu = None
    if not args.no_cpu_baseline:
        t_cpu, threads, rel, R, nz = cpu_baseline(rows, cols, vals, X, n, args.cpu_threads, Y, 16_000_000)
        cpu = cpu_entry(t_cpu, threads, nz, nnz, R, F, args.config)
        extra["parity_rel_l2_vs_cpu"] = rel
        extra["parity_rows"] = R
        extra["cpu_torch_sparse_mm"] = torch_sparse_cpu(rows, cols, vals, X, n, args.cpu_threads, 16_000_000)
    roofline = {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic_of(args.config), "kernel": kernel,
                "bytes_alg_per_launch": b_alg}
    config = {"workload": WORKLOADS[args.config], "n": n, "nnz": nnz, "F": F}
    return line_for(args, round(flops / (ms * 1e-3) / 1e9, 3), "GFLOP/s", ms, "fp32", config, roofline, cpu, extra)


def gcn_inputs(torch, cfg):
    """Config-4/5 graph, features, hot/cold table and layer graphs."""
    from tcc_amd import gcn
    from tcc_amd.graphs import make_features, make_graph

    n, F = cfg["n"], cfg["F"]
    t0 = time.time()
    rows, cols, _ = make_graph(4, device="cuda")
    X = make_features(n, F, cfg["seed"], device="cuda")
    table = gcn.FeatureTable(X, cols)
    g1, g2 = gcn.build_gcn_graphs(rows, cols, n, table.hot)
    torch.cuda.synchronize()
    print(f"[bench] graph n={n} nnz={rows.numel()} F={F}: generated and blocked in {time.time() - t0:.1f}s",
          file=sys.stderr, flush=True)
    return rows, cols, X, table, g1, g2


def packed_rows_step(torch, table, X, cols, g1, F, Y_fp32, cold_rows_used, args):
    """The same first-layer step with FeatureTable(packed=True): hot cache and
    host rows as packed TF32 rows (an option of this build; the headline
    keeps the reference's fp32 rows).  Checked against the fp32-row result."""
    from tcc_amd import gcn, swtcf

    ptable = gcn.FeatureTable(X, cols, packed=True)
    assert torch.equal(ptable.hot, table.hot)
    Yp = None

    def step():
        nonlocal Yp
        Yp = g1.aggregate(F, source=ptable.source)

    ms = timed(step, args.steps, args.warmup)
    torch.cuda.synchronize()
    rel = float((Yp - Y_fp32).norm() / Y_fp32.norm().clamp_min(1e-30))
    row_bytes = swtcf._lib.lib().tcc_tf32_packed_bytes(1, F)
    ptable.free()
    link = cold_rows_used * row_bytes
    return {"ms": round(ms, 4), "row_bytes": row_bytes, "cold_bytes": link,
            "host_link_GBps": round(link / (ms * 1e-3) / 1e9, 2), "rel_l2_vs_fp32_rows": rel}


def bench_mixed(args, torch, swtcf, cfg):
    """Config 4: the first-layer SpMM with hot rows from HBM and cold rows
    read zero-copy from pinned host memory."""
    n, F = cfg["n"], cfg["F"]
    rows, cols, X, table, g1, _ = gcn_inputs(torch, cfg)
    nnz = rows.numel()
    Y = None

    def step():
        nonlocal Y
        Y = g1.aggregate(F, source=table.source)

    ms = timed(step, args.steps, args.warmup)
    torch.cuda.synchronize()
    cold_edge = ~table.hot[cols.long()]
    hot_edges = int((~cold_edge).sum().item())
    cold_rows_used = int(torch.unique(cols[cold_edge]).numel())
    cold_bytes = 4.0 * F * cold_rows_used
    extra = {"hot_rows": table.n_hot, "hot_edges": hot_edges, "cold_edges": nnz - hot_edges,
             "bcsr_blocks": g1.bcsr.view.num_TCBlocks,
             "bcsc_blocks": g1.bcsc.view.num_TCBlocks if g1.bcsc is not None else 0,
             "host_link": {"cold_rows": cold_rows_used, "bytes_min": cold_bytes,
                           "achieved_GBps": round(cold_bytes / (ms * 1e-3) / 1e9, 2),
                           "peak_GBps": PCIE_PEAK_GBPS,
                           "bound_ms": round(cold_bytes / (PCIE_PEAK_GBPS * 1e9) * 1e3, 3)}}
    extra["packed_rows"] = packed_rows_step(torch, table, X, cols, g1, F, Y, cold_rows_used, args)
    cpu = None
    if not args.no_cpu_baseline:
        t_cpu, threads, rel, R, nz = cpu_baseline(rows, cols, None, X, n, args.cpu_threads, Y, 16_000_000)
        cpu = cpu_entry(t_cpu, threads, nz, nnz, R, F, 4)
        extra["parity_rel_l2_vs_cpu"] = rel
        extra["parity_rows"] = R
        extra["cpu_torch_sparse_mm"] = torch_sparse_cpu(rows, cols, None, X, n, args.cpu_threads, 16_000_000)
    # One launch (mixed_forward_kernel) interleaves the HBM-bound hot gather
    # with the scatter of cold rows read across the host link; the link bounds
    # it: the cold rows' bytes over PCIe Gen5 x16 (64 GB/s per direction).
    b_alg = bytes_alg(n, n, nnz, F)
    hbm_achieved = b_alg / (ms * 1e-3) / 1e9
    link_achieved = cold_bytes / (ms * 1e-3) / 1e9
    roofline = {"bound": "host_link", "achieved": round(link_achieved, 2), "peak": PCIE_PEAK_GBPS, "unit": "GB/s",
                "frac": round(link_achieved / PCIE_PEAK_GBPS, 4), "traffic": None,
                "kernel": "mixed_forward_kernel (gather_body<Mixed> + scatter_body<Mixed>)",
                "bytes_alg_per_launch": cold_bytes,
                "hbm": {"achieved": round(hbm_achieved, 2), "peak": HBM_PEAK_GBPS,
                        "frac": round(hbm_achieved / HBM_PEAK_GBPS, 4), "bytes_alg_per_launch": b_alg}}
    config = {"workload": WORKLOADS[4], "n": n, "nnz": nnz, "F": F}
    table.free()
    return line_for(args, round(2.0 * nnz * F / (ms * 1e-3) / 1e9, 3), "GFLOP/s", ms, "fp32", config, roofline,
                    cpu, extra)


def bench_gcn(args, torch, swtcf, cfg):
    """Config 5: one full-graph GCN training epoch per step, plus each
    layer's forward+backward time."""
    from tcc_amd import gcn

    n, F = cfg["n"], cfg["F"]
    hidden, classes = 256, 2
    rows, cols, X, table, g1, g2 = gcn_inputs(torch, cfg)
    nnz = rows.numel()
    torch.manual_seed(cfg["seed"])
    model = gcn.GCN(F, hidden, classes, dropout=0.0).cuda()
    labels = gcn.synthetic_labels(n, classes, cfg["seed"])
    opt = torch.optim.Adam(model.parameters(), lr=0.003)
    loss_fcn = gcn.cross_entropy
    losses = []

    def epoch():
        losses.append(gcn.train_epoch(model, g1, g2, table.source, labels, opt, loss_fcn))

    steps = max(1, min(args.steps, 10))
    warmup = max(1, min(args.warmup, 3))
    ms = timed(epoch, steps, warmup)
    first_loss, last_loss = float(losses[0].item()), float(losses[-1].item())

    g_h = torch.randn((n, hidden), device="cuda")
    g_c = torch.randn((n, classes), device="cuda")

    def layer1():
        model.zero_grad(set_to_none=True)
        model.conv1(g1, source=table.source).backward(g_h)

    x2 = torch.relu(model.conv1(g1, source=table.source)).detach().requires_grad_(True)

    def layer2():
        model.zero_grad(set_to_none=True)
        x2.grad = None
        model.conv_final(g2, x=x2).backward(g_c)

    l1 = timed(layer1, steps, warmup)
    l2 = timed(layer2, steps, warmup)
    # the same epoch over a packed TF32 feature table (an option; see packed_rows_step)
    ptable = gcn.FeatureTable(X, cols, packed=True)
    ms_packed = timed(lambda: gcn.train_epoch(model, g1, g2, ptable.source, labels, opt, loss_fcn), steps, warmup)
    ptable.free()
    extra = {"epoch": "TwoLayerFunction: mixed SpMM F=100 (one launch), relu(AX W1) and H W2 in one pass "
                      "(tcc_gcn_relu_forward), SpMM F=2; backward A^T SpMM F=2, then dW1 and dW2 in one pass "
                      "(tcc_gcn_relu_grad); cross-entropy, Adam",
             "layer_times": "each layer alone, through its own autograd function",
             "epoch_ms_packed_feature_rows": round(ms_packed, 4),
             "layer1_fwd_bwd_ms": round(l1, 4), "layer2_fwd_bwd_ms": round(l2, 4),
             "layer1": f"mixed SpMM F={F} (hot BCSR + cold BCSC) + GEMM {F}x{hidden}; backward dW GEMM",
             "layer2": f"A(XW): GEMM {hidden}x{classes}, BCSR SpMM F={classes}; backward A^T SpMM F={classes}, "
                       f"dW and dX GEMMs",
             "loss_first": first_loss, "loss_last": last_loss}
    config = {"workload": WORKLOADS[5], "n": n, "nnz": nnz, "F": F, "hidden": hidden, "classes": classes}
    table.free()
    line = line_for(args, round(ms, 4), "ms", ms, "fp32", config, None, None, extra, higher=False)
    line["steps"], line["warmup"] = steps, warmup
    return line


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no multi-GPU path",
              file=sys.stderr)
        return 2
    import torch

    from tcc_amd import swtcf
    from tcc_amd.graphs import CONFIGS

    assert torch.cuda.is_available(), "bench.py needs the GPU"
    torch.cuda.set_device(0)
    cfg = CONFIGS[args.config]
    if args.config in (1, 2, 3):
        line = bench_spmm(args, torch, swtcf, cfg)
    elif args.config == 4:
        line = bench_mixed(args, torch, swtcf, cfg)
    else:
        line = bench_gcn(args, torch, swtcf, cfg)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
