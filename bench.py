#!/usr/bin/env python3
"""Benchmark of the SWTCF / spmm_cnic hot path on one MI355X.

Default workload ("config 3", the north star's
target and the largest single-GPU configuration): R-MAT graph, 233k nodes,
114M nnz, sym-normalised fp32 values, X = N(0,1) [233k x 602]; one step = one
SpMM Y = A X over the whole graph with TF32 numerics, inputs resident in HBM
(the TF32 packing of X and the zero fill of Y are inside the step).  The same
run also times, under `extra`:
  config2  R-MAT 169k nodes, 1.17M nnz, F=128: forward BCSR SpMM
  config5  2-layer GCN (100 -> 256 -> 2, ReLU) on the config-4 graph: one
           full-graph training epoch, and each layer's forward+backward
Other configurations as the main line: --config 1 (uniform 4096 x 16/row,
F=32: SWTCF convert + SWTCF SpMM), 2, 4 (2.45M nodes, 61.9M nnz, F=100, top-20%
rows hot in HBM, the rest zero-copy from pinned host memory: mixed SpMM), 5.

Prints one JSON line.  SpMM configurations report GFLOP/s (2*nnz*F per
step) and their roofline: with the algorithmic bytes
4F(n_src+n_dst) + 8 nnz + 4(n_dst+1) and AI = flops / bytes, the roof is
min(157.3 TFLOP/s, AI * 8 TB/s); config 3 (AI 67.5) is bound by the fp32
roof, config 2 (AI 1.6) by HBM.  The counter-measured DRAM traffic of the
step's kernels (rocprofv3 FETCH_SIZE + WRITE_SIZE, profiles/) is reported
beside it.  The CPU baseline is the reference's own SpMM call,
torch.sparse.mm (train/tcgnn_conv_release.py:152), on the host cores over a
bounded sample of the same matrix; the oracle's CSR loop is timed beside it
and checks the GPU result on that sample.
"""
from __future__ import annotations

import argparse
import copy
import hashlib
import json
import os
import sys
import time
import warnings

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "SpMM GFLOP/s (2·nnz·F) + % HBM roofline; GCN layer fwd+bwd ms at 1 GPU"
HBM_PEAK_GBPS = 8000.0
FP32_PEAK_TFLOPS = 157.3  # MI355X fp32 (vector = matrix)
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
# The binary hybrid's remainder (9.8% of config 3's entries) takes 2 phases:
# config 3 step 4.76 ms against 4.99 with 4, 4.79 with 1 and 5.73 with 6.
BINARY_REST_PHASES = 2
# The same long-window (skewed) graphs hold a dense core once rows and
# columns are ordered by degree.  Config 3's values are sym-normalised,
# v_ij = r_i c_j with r = rowdeg^-1/2 and c = coldeg^-1/2, so the product
# is diag(r) P diag(c) X over the pattern P: steps (256 rows x 16 columns of
# the reordered matrix) holding at least BINARY_MIN_STEP_NNZ entries go to
# binary tiles on MFMA over 2^e TF32(c X) (fp16 where exact, else bf16
# halves), the rest to the phased gather of the packed TF32(c X) rows, each
# row sum scaled by r (tcc_coo_to_hybrid_scaled).  Measured at config 3
# (step ms): phased gather alone 17.35; valued split tiles (each TF32 value
# as two bf16, four bf16 products) 8.86 at 16 nnz a tile, groups of 8;
# binary tiles on dense MFMA with bf16 halves only 6.56 at 64 entries a
# 16-column step; with fp16 records, the tiles before the remainder, 5.52
# at 36 entries; on the 2:4 sparse MFMA over 32-column steps, 4.99 at 40
# entries and 768-step units, 4.55 with 1024-step units (the builder's
# defaults) after the launch-order and second-stream changes.  The valued hybrid
# is timed beside it under `extra`.
HUB_MIN_TILE_NNZ = 16
HUB_GROUP_BLOCKS = 8
BINARY_MIN_STEP_NNZ = 40
BINARY_GROUP_BLOCKS = 16
CPU_SAMPLE_NNZ = 16_000_000

WORKLOADS = {
    1: "config1: uniform 4096 nodes x 16 nnz/row, F=32, SWTCF convert + SWTCF SpMM",
    2: "config2: R-MAT (0.57,0.19,0.19) 169k nodes, 1.17M nnz, sym-normalised, F=128, forward BCSR SpMM",
    3: "config3: R-MAT (0.57,0.19,0.19) 233k nodes, 114M nnz, sym-normalised, F=602, SpMM (HBM-bound regime)",
    4: "config4: R-MAT 2.45M nodes, 61.9M nnz, F=100, top-20% rows hot in HBM, rest pinned host: mixed SpMM",
    5: "config5: 2-layer GCN 100->256->2 (ReLU, dropout 0, Adam 0.003) on the config-4 graph, full-graph epoch",
}


def parse(argv=None):
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=None,
                   help="timed steps (default: 500 for the microsecond configs 1-2, else 50)")
    p.add_argument("--warmup", type=int, default=None, help="untimed steps (default: 50 for configs 1-2, else 10)")
    p.add_argument("--config", type=int, default=3, choices=sorted(WORKLOADS))
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-extra", action="store_true",
                   help="config 3: skip the config-2 and config-5 timings under `extra`")
    p.add_argument("--cpu-threads", type=int, default=0, help="0 = all host cores")
    p.add_argument("--copy-calibration-mib", type=int, default=0,
                   help="first run one plain device copy of this many MiB (scale for rocprofv3 FETCH/WRITE_SIZE)")
    p.add_argument("--swtcf-ab", action="store_true",
                   help="SWTCF SpMM: VALU path against MFMA for dense tiles, synthetic tiles of k = 8..64 entries")
    p.add_argument("--swtcf-int8", action="store_true",
                   help="SWTCF SpMM on the config-3 graph at F = 128: fp32 X against int8 X")
    p.add_argument("--swtcf-step", choices=("fp32", "int8"), default=None,
                   help="configs 2-3: the step is launchSWTCFSpMM (fp32 X) or launchSWTCFSpMMQuantized (int8 X "
                        "with per-row scales) over the SWTCF (S = 16) of the config's graph at the reference's "
                        "F = 128 (for counter runs of the SWTCF SpMM)")
    p.add_argument("--no-swtcf-plans", action="store_true",
                   help="with --swtcf-step: the SWTCF kernel on every launch (tcc_swtcf_set_plans(0)), not the "
                        "plan later launches over one large matrix take")
    p.add_argument("--atomic-probe-mib", type=int, default=0,
                   help="time tcc_calibration_atomic over a buffer of this many MiB (rows of 128 floats, 64-float "
                        "segments at random rows: the SWTCF SpMM's output pattern) and print one JSON line")
    p.add_argument("--profile-convert", action="store_true",
                   help="configs 1-3: time only convertCOOToSWTCF (S = 16), warmup + steps conversions, and print "
                        "one JSON line (for rocprofv3 runs of the converter)")
    p.add_argument("--convert-order", choices=("both", "dst-src", "shuffled"), default="both",
                   help="with --profile-convert: time the COO in the generator's (dst, src) order, the same COO "
                        "shuffled (every digit of the sort runs), or both")
    p.add_argument("--no-hybrid", action="store_true",
                   help="config 3: the phased packed gather alone (no dense hub tiles), the path before them")
    p.add_argument("--profile-step", action="store_true",
                   help="for counter runs: only the timed step's kernels run (warmup + steps times); no CPU "
                        "baseline, comparisons, conversions or extra configs")
    args = p.parse_args(argv)
    if args.profile_step:
        args.no_cpu_baseline = args.no_extra = True
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


def roofline(flops, b_alg, ms, traffic, kernel):
    """The metric's roofline: AI = flops / algorithmic bytes, roof =
    min(fp32 peak, AI * HBM peak).  `achieved` is the step's rate in the
    binding roof's unit, so frac = achieved / peak = (flops/t) / roof.
    `traffic` is the counter-measured HBM bytes of the step's kernels."""
    t = ms * 1e-3
    ai = flops / b_alg
    if FP32_PEAK_TFLOPS * 1e12 <= ai * HBM_PEAK_GBPS * 1e9:
        bound, achieved, peak, unit = "mfma", flops / t / 1e12, FP32_PEAK_TFLOPS, "TFLOP/s"
    else:
        bound, achieved, peak, unit = "hbm", b_alg / t / 1e9, HBM_PEAK_GBPS, "GB/s"
    r = {"bound": bound, "achieved": round(achieved, 4), "peak": peak, "unit": unit, "frac": round(achieved / peak, 4),
         "traffic": None if traffic is None else traffic["hbm_bytes_per_launch"], "kernel": kernel,
         "arith_intensity": round(ai, 3), "bytes_alg_per_launch": b_alg, "flops_per_launch": flops,
         "roof": "min(157.3 TFLOP/s fp32, AI x 8 TB/s)"}
    if bound == "mfma":
        r["fp32"] = ("fp32 peak 157.3 TFLOP/s, the roof for this metric; which unit each kernel uses "
                     "(VALU fp32 FMA, fp32 MFMA, bf16 MFMA over split TF32) is in `kernel`")
    r["hbm_fraction_alg"] = round(b_alg / t / 1e9 / HBM_PEAK_GBPS, 4)
    if traffic is not None:
        gbps = traffic["hbm_bytes_per_launch"] / t / 1e9
        r["l2_fabric_traffic"] = {
            "GBps": round(gbps, 1), "bytes_per_step": traffic["hbm_bytes_per_launch"], "source": traffic["file"],
            "what": "rocprofv3 FETCH_SIZE + WRITE_SIZE of the step's kernels (scaled by a 1 GiB copy) over this "
                    "run's event-timed step: requests from the L2 to the fabric, Infinity Cache hits included, "
                    "so re-reads of rows count as often as they are fetched; not an efficiency figure (the "
                    "roofline fraction is)"}
    return r


def _sha16(path):
    with open(os.path.join(ROOT, path), "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()[:16]


def traffic_of(config):
    """Counter-measured HBM bytes per step from profiles/traffic_config<N>.json,
    only when the kernel sources it was measured on are the ones built now."""
    name = f"profiles/traffic_config{config}.json"
    path = os.path.join(ROOT, name)
    if not os.path.exists(path):
        return None
    with open(path) as f:
        d = json.load(f)
    srcs = d.get("sources")
    if not srcs or any(_sha16(p) != h for p, h in srcs.items()):
        return None  # measured on other kernel sources
    return {"hbm_bytes_per_launch": d["hbm_bytes_per_launch"], "file": name}


def csr_sample(rows, cols, vals, n, max_nnz):
    """The leading rows of the matrix holding at most max_nnz nonzeros (the
    whole matrix when it is smaller), as CSR numpy arrays."""
    import numpy as np

    from tcc_amd.graphs import to_csr_numpy

    rowptr, colind, v = to_csr_numpy(rows, cols, n, vals)
    R = max(1, min(n, int(np.searchsorted(rowptr, max_nnz, side="right")) - 1))
    nz = int(rowptr[R])
    return (R, nz, np.ascontiguousarray(rowptr[: R + 1]), np.ascontiguousarray(colind[:nz]),
            None if v is None else np.ascontiguousarray(v[:nz]))


def oracle_cpu(sample, X, threads, Y_gpu):
    """The oracle's CSR SpMM (OpenMP, fp64 accumulation of TF32-rounded
    inputs) over the sample: median of 5 after 1 warm-up; also the parity
    check of the GPU result on those rows (rel-L2)."""
    import numpy as np

    import oracle

    R, nz, rp, ci, vv = sample
    Xc = X.cpu().numpy()
    oracle.csr_spmm(rp, ci, vv, Xc, use_tf32=True, threads=threads)
    ts, Y = [], None
    for _ in range(5):
        t0 = time.perf_counter()
        Y = oracle.csr_spmm(rp, ci, vv, Xc, use_tf32=True, threads=threads)
        ts.append(time.perf_counter() - t0)
    t = sorted(ts)[len(ts) // 2]
    yg = Y_gpu[:R].cpu().numpy().astype(np.float64)
    rel = float(np.linalg.norm(yg - Y) / max(np.linalg.norm(Y), 1e-30))
    F = X.shape[1]
    return {"value": round(2.0 * nz * F / t / 1e9, 3), "unit": "GFLOP/s", "cores": threads, "ms": round(t * 1e3, 3),
            "what": "oracle CSR SpMM (fp64 accumulation of TF32-rounded inputs, OpenMP over rows), same sample, "
                    "median of 5 after 1 warm-up"}, rel


def torch_sparse_cpu(sample, X, n, threads):
    """The reference's own SpMM call, torch.sparse.mm (train/tcgnn_conv_release.py:152),
    on the host cores in fp32 with a CSR tensor over the sample: median of 5
    after 1 warm-up.  Returns seconds."""
    import numpy as np
    import torch

    R, nz, rp, ci, vv = sample
    vv = np.ones(nz, np.float32) if vv is None else np.asarray(vv, np.float32)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")  # "sparse CSR support is in beta"
        A = torch.sparse_csr_tensor(torch.from_numpy(rp.astype(np.int64)), torch.from_numpy(ci.astype(np.int64)),
                                    torch.from_numpy(vv), size=(R, n))
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
    return sorted(ts)[len(ts) // 2]


def cpu_baselines(args, rows, cols, vals, X, n, Y_gpu, config, extra):
    """cpu_baseline = torch.sparse.mm over the sample; the oracle loop and
    the parity of the GPU result on the sample go to `extra`."""
    threads = args.cpu_threads or os.cpu_count() or 1
    sample = csr_sample(rows, cols, vals, n, CPU_SAMPLE_NNZ)
    R, nz = sample[0], sample[1]
    nnz, F = rows.numel(), X.shape[1]
    t = torch_sparse_cpu(sample, X, n, threads)
    what = (f"whole config-{config} matrix ({nnz} nnz, F={F})" if nz == nnz else
            f"rows 0..{R - 1} of config {config} ({nz} of {nnz} nnz, F={F})")
    cpu = {"value": round(2.0 * nz * F / t / 1e9, 3), "unit": "GFLOP/s", "cores": threads, "kind": "reference",
           "sample": f"{what}; torch.sparse.mm (CSR, fp32), the reference's own SpMM call "
                     f"(train/tcgnn_conv_release.py:152), median of 5 after 1 warm-up",
           "ms": round(t * 1e3, 3)}
    o, rel = oracle_cpu(sample, X, threads, Y_gpu)
    extra["cpu_oracle"] = o
    extra["parity_rel_l2_vs_oracle"] = rel
    extra["parity_rows"] = R
    return cpu


def timed(step, steps, warmup):
    """Mean ms per step over `steps` after `warmup`, timed with HIP events on
    the current stream (every launch of the step goes to that stream)."""
    return timed_stats(step, steps, warmup)[0]


def timed_stats(step, steps, warmup):
    """(mean, median) ms per step, as `timed`, with an event between steps
    (the reference's drivers report both, swtcf_spmm_main.cu:203-247); the
    mean is first to last event over `steps`."""
    import statistics

    import torch

    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    ev[0].record(stream)
    for i in range(steps):
        step()
        ev[i + 1].record(stream)
    torch.cuda.synchronize()
    per = [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]
    return ev[0].elapsed_time(ev[steps]) / steps, statistics.median(per)


def graph_step_ms(torch, step, k):
    """ms per step of `k` steps captured in one HIP graph (torch.cuda.graph,
    after warm-up launches on a side stream) and replayed: launch-bound
    steps without the Python launch between them."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(k):
            step()
    ms = timed(g.replay, 20, 3) / k
    del g
    return ms


def copy_calibration(mib):
    """One calibration_copy_kernel dispatch reading and writing exactly `mib`
    MiB (tcc_calibration_copy), after which the source is evicted from the
    caches by writing a second buffer of the same size."""
    import torch

    from tcc_amd import _lib

    nfl = mib * (1 << 20) // 4
    a_src = torch.ones(nfl, device="cuda")
    a_dst = torch.empty_like(a_src)
    a_dst.fill_(2.0)  # evicts a_src from the L2 and the last-level cache
    torch.cuda.synchronize()
    _lib.check(_lib.lib().tcc_calibration_copy(a_dst.data_ptr(), a_src.data_ptr(), nfl * 4,
                                               torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    del a_src, a_dst


def line_for(args, value, unit, ms, dtype, config, roof, cpu, extra, higher=True, median=None):
    return {
        "metric": METRIC, "value": value, "unit": unit, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 5), "median_ms_per_step": None if median is None else round(median, 5),
        "higher_is_better": higher, "scaling": "weak", "vs_baseline": None,
        "dtype": dtype, "data": "synthetic (seeded generator, see tcc_amd/graphs.py)", "config": config,
        "roofline": roof, "cpu_baseline": cpu, "extra": extra,
    }


PLAN_KINDS = {
    2: "the BCSR gather of the matrix's pattern (a plain BCSR: rows are gathered 7.3 times on average)",
    3: "binary hub tiles on the sparse MFMA + gathered remainder of the matrix's pattern",
}


def swtcf_plan_timings(torch, swtcf, m, n, nnz, config):
    """launchSWTCFSpMM (and launchSWTCFSpMMQuantized, int8 X with per-row
    scales, src/swtcf_spmm.cu:469-502) on the config's graph at the
    reference's F = 128, S = 16: the SWTCF kernel (plans off) and the kept
    plan (the second call on the matrix builds it), Y += A X without
    zeroing Y between launches, as the reference times it
    (swtcf_spmm_main.cu:203-247 sets Y once)."""
    L = swtcf._lib.lib()
    F = 128
    X = torch.randn((n, F), device="cuda", generator=torch.Generator(device="cuda").manual_seed(11))
    Y = torch.zeros((n, F), device="cuda")
    step = lambda: swtcf.launchSWTCFSpMM(m, X, Y, 12)
    scale = X.abs().amax(dim=1).clamp_min(1e-30) / 127.0
    q = torch.round(X / scale[:, None]).clamp(-127, 127).to(torch.int8).contiguous()
    src_global = torch.arange(n, dtype=torch.int32, device="cuda")
    qstep = lambda: swtcf.launchSWTCFSpMMQuantized(m, q, scale.contiguous(), src_global, Y, 12)
    reps = (20, 3) if config == 2 else (3, 1)
    L.tcc_swtcf_set_plans(0)
    kernel_ms = timed(step, *reps)
    int8_kernel_ms = timed(qstep, *reps)
    L.tcc_swtcf_set_plans(1)
    L.tcc_swtcf_release_plans()
    built0 = L.tcc_swtcf_plans_built()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    step()  # first sighting: the kernel
    step()  # second: builds the plan and runs it
    torch.cuda.synchronize()
    first_two_ms = (time.perf_counter() - t0) * 1e3
    assert L.tcc_swtcf_plans_built() == built0 + 1
    plan_ms = timed(step, 20, 2)
    # int8 X: the same plan, X dequantized into its buffer first
    int8_plan_ms = timed(qstep, 20, 2)
    assert L.tcc_swtcf_plans_built() == built0 + 1
    L.tcc_swtcf_release_plans()
    gf = lambda ms: round(2.0 * nnz * F / (ms * 1e-3) / 1e9, 3)
    return {"F": F, "S": 16, "kernel_ms": round(kernel_ms, 4), "kernel_gflops": gf(kernel_ms),
            "int8_kernel_ms": round(int8_kernel_ms, 4), "int8_kernel_gflops": gf(int8_kernel_ms),
            "plan_ms": round(plan_ms, 4), "plan_gflops": gf(plan_ms),
            "int8_plan_ms": round(int8_plan_ms, 4), "int8_plan_gflops": gf(int8_plan_ms),
            "first_two_calls_ms": round(first_two_ms, 2),
            "plan": PLAN_KINDS[config] + ", built on the second call that finds the same arrays (device hash "
                                         "each call)",
            "X_bytes_fp32": 4 * n * F, "X_bytes_int8": n * F + 4 * n}


def bench_swtcf_ab(args, torch, swtcf):
    """SWTCF SpMM, VALU path against fp32 MFMA for dense tiles
    (tcc_swtcf_spmm_mfma), on synthetic matrices whose 8x8 tiles all hold k
    entries: 2048 rows x 2048 windows of 8 columns, every row holding k/8
    random columns of every window (so each window's 256 tiles hold k
    entries), F = 128, tcThreshold 0 (TF32 X on both paths)."""
    R, CW, F = 2048, 2048, 128
    out = {"metric": "SWTCF SpMM ms, VALU vs MFMA for tiles of k entries", "rows": R, "windows": CW, "F": F,
           "tiles": R // 8 * CW, "steps": args.steps, "warmup": args.warmup, "per_k": []}
    gen = torch.Generator(device="cuda").manual_seed(7)
    X = torch.randn((8 * CW, F), device="cuda", generator=gen)
    for k in (8, 16, 24, 32, 40, 48, 56, 64):
        pick = torch.rand((R, CW, 8), device="cuda", generator=gen).argsort(dim=2)[:, :, : k // 8]
        dst = torch.arange(R, device="cuda", dtype=torch.int32).view(R, 1, 1).expand(R, CW, k // 8)
        src = (torch.arange(CW, device="cuda", dtype=torch.int32).view(1, CW, 1) * 8 + pick.to(torch.int32))
        order = torch.argsort(dst.reshape(-1).to(torch.int64) * (8 * CW) + src.reshape(-1))
        d32 = dst.reshape(-1)[order].contiguous()
        s32 = src.reshape(-1)[order].contiguous()
        nnz = d32.numel()
        m = swtcf.DeviceSWTCFMatrix(R, 8 * CW, nnz, 16)
        ws = swtcf.SWTCFConvertWorkspace(nnz, 8 * CW, 16)
        swtcf.convertCOOToSWTCF(d32, s32, nnz, m, ws)
        assert ws.device_error() == 0
        Ya = torch.zeros((R, F), device="cuda")
        Yb = torch.zeros((R, F), device="cuda")
        swtcf.swtcf_spmm_mfma(m, X, Ya, 0, 65)
        swtcf.swtcf_spmm_mfma(m, X, Yb, 0, k)
        torch.cuda.synchronize()
        diff = ((Ya.double() - Yb.double()).norm() / Ya.double().norm()).item()
        t_valu = timed(lambda: swtcf.swtcf_spmm_mfma(m, X, Ya, 0, 65), args.steps, args.warmup)
        t_mfma = timed(lambda: swtcf.swtcf_spmm_mfma(m, X, Yb, 0, k), args.steps, args.warmup)
        out["per_k"].append({"k": k, "nnz": nnz, "valu_ms": round(t_valu, 4), "mfma_ms": round(t_mfma, 4),
                             "mfma_over_valu": round(t_mfma / t_valu, 3), "rel_l2_mfma_vs_valu": diff})
        print(f"[bench] swtcf A/B k={k}: VALU {t_valu:.4f} ms, MFMA {t_mfma:.4f} ms", file=sys.stderr, flush=True)
        del m, ws, Ya, Yb, pick, dst, src, order, d32, s32
        torch.cuda.empty_cache()
    # the benchmark graphs at F = 128, tcThreshold 12: VALU, then MFMA for
    # tiles of >= 12 (the reference's tensor-core threshold) and >= 32
    from tcc_amd.graphs import CONFIGS, make_graph

    out["graphs"] = []
    for c in (1, 2, 3):
        n = CONFIGS[c]["n"]
        rows, cols, _ = make_graph(c, device="cuda")
        r32 = rows.to(torch.int32).contiguous()
        c32 = cols.to(torch.int32).contiguous()
        nnz = rows.numel()
        del rows, cols
        m = swtcf.DeviceSWTCFMatrix(n, n, nnz, 16)
        ws = swtcf.SWTCFConvertWorkspace(nnz, n, 16)
        swtcf.convertCOOToSWTCF(r32, c32, nnz, m, ws)
        assert ws.device_error() == 0
        del ws
        Xg = torch.randn((n, F), device="cuda", generator=gen)
        Y = torch.zeros((n, F), device="cuda")
        steps, warmup = (args.steps, args.warmup) if c == 3 else (10 * args.steps, 10 * args.warmup)
        e = {"config": c, "n": n, "nnz": nnz}
        for mf in (65, 12, 32):
            e[f"ms_mfma_ge_{mf}" if mf <= 64 else "ms_valu"] = round(
                timed(lambda: swtcf.swtcf_spmm_mfma(m, Xg, Y, 12, mf), steps, warmup), 4)
        out["graphs"].append(e)
        print(f"[bench] swtcf A/B config {c}: {e}", file=sys.stderr, flush=True)
        del m, Xg, Y, r32, c32
        torch.cuda.empty_cache()
    return out


def bench_swtcf_int8(args, torch, swtcf):
    """launchSWTCFSpMMQuantized (int8 X, per-row scales) against
    launchSWTCFSpMM (fp32 X) on the config-3 graph at the reference's
    F = 128, tcThreshold 12."""
    from tcc_amd.graphs import CONFIGS, make_graph

    n = CONFIGS[3]["n"]
    rows, cols, _ = make_graph(3, device="cuda")
    r32 = rows.to(torch.int32).contiguous()
    c32 = cols.to(torch.int32).contiguous()
    nnz = rows.numel()
    del rows, cols
    m = swtcf.DeviceSWTCFMatrix(n, n, nnz, 16)
    ws = swtcf.SWTCFConvertWorkspace(nnz, n, 16)
    swtcf.convertCOOToSWTCF(r32, c32, nnz, m, ws)
    assert ws.device_error() == 0
    del ws
    gen = torch.Generator(device="cuda").manual_seed(11)
    X = torch.randn((n, 128), device="cuda", generator=gen)
    scales = X.abs().amax(dim=1).clamp_min(1e-30) / 127.0
    q = torch.round(X / scales[:, None]).clamp(-127, 127).to(torch.int8).contiguous()
    srcGlobal = torch.arange(n, device="cuda", dtype=torch.int32)
    Yf = torch.zeros((n, 128), device="cuda")
    Yq = torch.zeros((n, 128), device="cuda")
    t_f = timed(lambda: swtcf.launchSWTCFSpMM(m, X, Yf, 12), args.steps, args.warmup)
    t_q = timed(lambda: swtcf.launchSWTCFSpMMQuantized(m, q, scales, srcGlobal, Yq, 12), args.steps, args.warmup)
    Yf.zero_()
    Yq.zero_()
    swtcf.launchSWTCFSpMM(m, (q.float() * scales[:, None]).contiguous(), Yf, 12)
    swtcf.launchSWTCFSpMMQuantized(m, q, scales, srcGlobal, Yq, 12)
    torch.cuda.synchronize()
    diff = ((Yq.double() - Yf.double()).norm() / Yf.double().norm()).item()
    flops = 2.0 * nnz * 128
    return {"metric": "SWTCF SpMM ms at F = 128, fp32 X vs int8 X", "n": n, "nnz": nnz, "F": 128,
            "steps": args.steps, "warmup": args.warmup, "fp32_ms": round(t_f, 4), "int8_ms": round(t_q, 4),
            "fp32_GFLOPs": round(flops / t_f / 1e6, 1), "int8_GFLOPs": round(flops / t_q / 1e6, 1),
            "X_bytes_fp32": n * 128 * 4, "X_bytes_int8": n * 128 + 4 * n,
            "rel_l2_int8_vs_fp32_on_dequantized_X": diff}


def bench_convert(args, torch, swtcf, cfg):
    """convertCOOToSWTCF (S = 16) of the config's COO alone: warmup + steps
    conversions, the timed ones between HIP events."""
    from tcc_amd.graphs import make_graph

    if args.config not in (1, 2, 3):
        raise SystemExit("--profile-convert takes configs 1-3")
    n = cfg["n"]
    rows, cols, _ = make_graph(args.config, device="cuda")
    r32 = rows.to(torch.int32).contiguous()
    c32 = cols.to(torch.int32).contiguous()
    nnz = rows.numel()
    del rows, cols
    m = swtcf.DeviceSWTCFMatrix(n, n, nnz, 16)
    ws = swtcf.SWTCFConvertWorkspace(nnz, n, 16)
    out = {"metric": "convertCOOToSWTCF ms (S = 16)", "unit": "ms", "steps": args.steps, "warmup": args.warmup,
           "config": {"workload": WORKLOADS[args.config], "n": n, "nnz": nnz}}
    if args.convert_order in ("both", "dst-src"):
        # the generator lists the COO in (dst, src) order: the sort's sw digits alone order it
        ms = timed(lambda: swtcf.convertCOOToSWTCF(r32, c32, nnz, m, ws), args.steps, args.warmup)
        assert ws.device_error() == 0
        out.update(value=round(ms, 4), gedges_per_s=round(nnz / ms / 1e6, 3), input_order="(dst, src)")
    if args.convert_order in ("both", "shuffled"):
        # the same COO in random order: every digit of the sort runs
        perm = torch.randperm(nnz, device="cuda", generator=torch.Generator(device="cuda").manual_seed(5))
        r32, c32 = r32[perm].contiguous(), c32[perm].contiguous()
        del perm
        ms_s = timed(lambda: swtcf.convertCOOToSWTCF(r32, c32, nnz, m, ws), args.steps, args.warmup)
        assert ws.device_error() == 0
        key = "shuffled_ms" if "value" in out else "value"
        out[key] = round(ms_s, 4)
        out["shuffled_gedges_per_s"] = round(nnz / ms_s / 1e6, 3)
        if key == "value":
            out["input_order"] = "shuffled"
    return out


def extension_timings(torch, swtcf, r32, c32, n, F, X):
    """Config 3 through the reference's own entry point, spmm_cnic's
    forward_tensorcore (train/tcgnn_conv_release.py:124-130), called
    unchanged on the whole graph as a BCSR (values not read, as the
    reference's kernels read none; an empty BCSC): the default path (x packed
    to TF32 rows when rows are gathered >= 16 times) and a per-graph plan
    (set_graph_plans), with the plan's one-time build."""
    sys.path.insert(0, os.path.join(ROOT, "tcc_amd"))
    try:
        import spmm_cnic
    finally:
        sys.path.pop(0)

    import numpy as np

    def tensors(d, kind):
        def dev(arr):
            arr = np.ascontiguousarray(arr)
            view = np.int32 if arr.dtype == np.uint32 else (np.int64 if arr.dtype == np.uint64 else arr.dtype)
            return torch.from_numpy(arr.view(view)).cuda()

        w, i = ("rowWindowOffset", "sparseA2B") if kind == "bcsr" else ("colWindowOffset", "sparseA2C")
        nw = d["num_rowWindows"] if kind == "bcsr" else d["num_colWindows"]
        return [d["num_rows"], d["num_cols"], d["nnz"], d["num_TCBlocks"], nw, dev(d[w]), dev(d["tcOffset"]),
                dev(d[i]), dev(d["tcLocalBit"]), torch.zeros(1, device="cuda")]

    A = swtcf.coo_to_bcsr(r32, c32, None, n, n)
    B = swtcf.coo_to_bcsc(r32[:0], c32[:0], None, n, n)
    args = tensors(A.to_host(), "bcsr") + tensors(B.to_host(), "bcsc")
    A.release()
    B.release()
    x = X.flatten()
    flops = 2.0 * r32.numel() * F
    out = {"entry": "spmm_cnic.forward_tensorcore (Python-caller form), whole graph as BCSR, empty BCSC"}

    def step():
        spmm_cnic.forward_tensorcore(*args, F, x)
        spmm_cnic.freeMatC()

    spmm_cnic.set_graph_plans(0)
    try:
        ms = timed(step, 10, 2)
        out["packed_x_ms"] = round(ms, 4)
        out["packed_x_GFLOPs"] = round(flops / ms / 1e6, 1)
        # the default (automatic) plans, as an unchanged caller gets them:
        # the first call runs the packed gather and hashes the arrays, the
        # second builds the plan, later calls run it
        spmm_cnic.set_graph_plans(-1)
        spmm_cnic.release_plans()
        calls = []
        for _ in range(2):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            step()
            torch.cuda.synchronize()
            calls.append(round((time.perf_counter() - t0) * 1e3, 2))
        out["auto_first_call_ms"], out["auto_second_call_ms"] = calls
        ms = timed(step, 20, 2)
        out["plan_ms"] = round(ms, 4)
        out["plan_GFLOPs"] = round(flops / ms / 1e6, 1)
        out["plans"] = ("automatic: a device hash of the BCSR arrays each call; the second call that finds the "
                        "same arrays builds the plan (binary tiles + gather), later calls run it")
    finally:
        spmm_cnic.set_graph_plans(-1)
        spmm_cnic.release_plans()
    return out


def bench_swtcf_step(args, torch, swtcf, cfg):
    """Configs 2-3 (--swtcf-step): one launchSWTCFSpMM (or its int8 form) per
    step over the SWTCF (S = 16) of the config's graph at F = 128, Y += A X
    without zeroing Y between steps, as the reference's driver times it
    (swtcf_spmm_main.cu:203-247)."""
    from tcc_amd.graphs import make_graph

    n, F = cfg["n"], 128
    rows, cols, _ = make_graph(args.config, device="cuda")
    r32 = rows.to(torch.int32).contiguous()
    c32 = cols.to(torch.int32).contiguous()
    nnz = rows.numel()
    del rows, cols
    m = swtcf.DeviceSWTCFMatrix(n, n, nnz, 16)
    ws = swtcf.SWTCFConvertWorkspace(nnz, n, 16)
    swtcf.convertCOOToSWTCF(r32, c32, nnz, m, ws)
    assert ws.device_error() == 0
    del ws
    X = torch.randn((n, F), device="cuda", generator=torch.Generator(device="cuda").manual_seed(11))
    Y = torch.zeros((n, F), device="cuda")
    through = ("swtcf_spmm_kernel" if args.no_swtcf_plans else
               "its plan from the second call on: " + PLAN_KINDS[args.config])
    if args.swtcf_step == "fp32":
        step = lambda: swtcf.launchSWTCFSpMM(m, X, Y, 12)
        kernel = f"launchSWTCFSpMM, fp32 X: {through}"
    else:
        scales = X.abs().amax(dim=1).clamp_min(1e-30) / 127.0
        q = torch.round(X / scales[:, None]).clamp(-127, 127).to(torch.int8).contiguous()
        src_global = torch.arange(n, dtype=torch.int32, device="cuda")
        step = lambda: swtcf.launchSWTCFSpMMQuantized(m, q, scales.contiguous(), src_global, Y, 12)
        kernel = f"launchSWTCFSpMMQuantized, int8 X, per-row scales: {through}"
    if args.copy_calibration_mib:
        copy_calibration(args.copy_calibration_mib)
    ms, median = timed_stats(step, args.steps, args.warmup)
    flops = 2.0 * nnz * F
    roof = roofline(flops, bytes_alg(n, n, nnz, F), ms, None, kernel)
    config = {"workload": WORKLOADS[args.config] + "; SWTCF SpMM at F = 128, S = 16", "n": n, "nnz": nnz, "F": F}
    return line_for(args, round(flops / (ms * 1e-3) / 1e9, 3), "GFLOP/s", ms, "fp32" if args.swtcf_step == "fp32"
                    else "int8", config, roof, None, {"path": kernel}, median=median)


def atomic_probe(args, torch, swtcf):
    """tcc_calibration_atomic over a buffer of args.atomic_probe_mib MiB:
    atomics per second for 64-float segments at random rows (rows of 128
    floats, as the SWTCF SpMM's Y at F = 128)."""
    from tcc_amd import _lib

    rows = max(1, args.atomic_probe_mib * (1 << 20) // 512)
    dst = torch.zeros(rows * 128, device="cuda")
    waves = 1 << 22  # 268M atomic adds
    st = torch.cuda.current_stream().cuda_stream
    step = lambda: _lib.check(_lib.lib().tcc_calibration_atomic(dst.data_ptr(), rows, 128, waves, st))
    ms, median = timed_stats(step, args.steps, args.warmup)
    n = waves * 64
    return {"metric": "fp32 atomic adds per second (tcc_calibration_atomic)", "buffer_mib": args.atomic_probe_mib,
            "rows": rows, "atomics_per_launch": n, "ms": round(ms, 4), "median_ms": round(median, 4),
            "G_atomics_per_s": round(n / (ms * 1e-3) / 1e9, 2),
            "payload_GBps": round(4.0 * n / (ms * 1e-3) / 1e9, 1),
            "pattern": "wave w: 64 consecutive floats (256 B) of a pseudo-random row of 128 floats, one per lane"}


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
        perm = torch.randperm(nnz, device="cuda", generator=torch.Generator(device="cuda").manual_seed(5))
        rs32, cs32 = r32[perm].contiguous(), c32[perm].contiguous()
        conv_s = timed(lambda: swtcf.convertCOOToSWTCF(rs32, cs32, nnz, m, ws), 20, 2)
        assert ws.device_error() == 0
        extra["convert_shuffled_ms"] = round(conv_s, 4)
        # the matrix of the COO in its own order, for the SpMM below
        swtcf.convertCOOToSWTCF(r32, c32, nnz, m, ws)
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
        H = None
        if per_window >= PHASE_MIN_BLOCKS_PER_WINDOW:
            # long windows: the phased BCSR of the same COO, built once
            t_p = time.perf_counter()
            Ap = swtcf.coo_to_bcsr(r32, c32, vals, n, n, phases=PHASES)
            torch.cuda.synchronize()
            extra["phased_build_ms"] = round((time.perf_counter() - t_p) * 1e3, 3)
            extra["phases"] = PHASES
            A.release()
            A = Ap
        if per_window >= PHASE_MIN_BLOCKS_PER_WINDOW and not args.no_hybrid:
            # ... and the hybrid: binary hub tiles on MFMA + the phased gather
            # of the rest, the sym-normalised values as row and column scales
            from tcc_amd.graphs import sym_norm_scales

            rs, cs = sym_norm_scales(rows, cols, n)
            # the scales reproduce the values: v_ij against fp32(r_i c_j)
            fact = ((rs[rows] * cs[cols] - vals).abs() / vals.abs()).max().item()
            t_h = time.perf_counter()
            H = swtcf.coo_to_hybrid_scaled(r32, c32, n, n, rs, cs, min_step_nnz=BINARY_MIN_STEP_NNZ,
                                           group_blocks=BINARY_GROUP_BLOCKS, phases=BINARY_REST_PHASES)
            torch.cuda.synchronize()
            extra["hybrid_build_ms"] = round((time.perf_counter() - t_h) * 1e3, 3)
            t = H.view.tiles
            extra["hub"] = {"format": "binary patterns of 32-row by 32-column tiles as 2:4 operands of "
                                      "v_smfmac_f32_32x32x32_f16 against fp16 2^e TF32(c X) where exact (else "
                                      "_bf16 against its bf16 halves), a second layer where a group of four "
                                      "columns holds more than two entries; rows scaled by 2^-e r",
                            "min_step_nnz": BINARY_MIN_STEP_NNZ, "group_blocks": t.group_blocks,
                            "sub_steps": t.num_steps, "units": t.num_units, "partial_units": t.num_partial_units,
                            "hub_cols": t.hub_cols, "tile_nnz": t.nnz, "tile_nnz_frac": round(t.nnz / nnz, 4),
                            "rest_blocks": H.rest.view.num_TCBlocks,
                            # one sparse f16 MFMA (32x32x32, 2:4) a tile and 32-feature slice (two
                            # bf16 for a bf16 record): dense-equivalent flops, zeros included
                            "smfmac_dense_equiv_flops_fp16_records": 1024.0 * t.group_blocks * t.num_steps
                            * (-(-F // 32) * 32),
                            "values_as_scales_max_rel_diff": fact}
        Y = torch.empty((A.out_windows * 8, F), device="cuda")
        phased = f" over the {A.phases}-phase BCSR (Y zero-filled first)" if A.phases > 1 else ""
        if H is not None:
            if not args.profile_step:
                # the phased gather alone and the valued hybrid (each TF32
                # value split into two bf16 tiles), timed in the same run
                buf = torch.empty(swtcf._lib.lib().tcc_tf32_packed_bytes(n, F) + 16, dtype=torch.uint8,
                                  device="cuda")
                extra["phased_gather_ms"] = round(
                    timed(lambda: swtcf.bcsr_spmm_packed(A, swtcf.tf32_pack(X, out=buf), F, Y), 10, 2), 4)
                del buf
                Hv = swtcf.coo_to_hybrid(r32, c32, vals, n, n, min_tile_nnz=HUB_MIN_TILE_NNZ,
                                         group_blocks=HUB_GROUP_BLOCKS, tile_format=swtcf.TILES_BF16X2,
                                         phases=PHASES)
                Yv = torch.empty((Hv.out_rows, F), device="cuda")
                vws = torch.empty(Hv.workspace_bytes(F) + 16, dtype=torch.uint8, device="cuda")
                extra["valued_hybrid_ms"] = round(timed(lambda: swtcf.hybrid_spmm(Hv, X, Yv, workspace=vws), 10, 2), 4)
                extra["valued_hybrid"] = (f"split-TF32 value tiles (>= {HUB_MIN_TILE_NNZ} nnz, groups of "
                                          f"{HUB_GROUP_BLOCKS}) + packed gather of the valued remainder")
                Hv.release()
                del Yv, vws
            A.release()
            Y = torch.empty((H.out_rows, F), device="cuda")
            hws = torch.empty(H.workspace_bytes(F) + 16, dtype=torch.uint8, device="cuda")

            def step():
                swtcf.hybrid_spmm(H, X, Y, workspace=hws)

            G = H.view.tiles.group_blocks
            kernel = (f"hub_tiles_binary_kernel<{G}, {1 if G == 16 else 2}, 4> (2:4 sparse f16 MFMA "
                      "32x32x32 over 2^e TF32(c X), bf16 halves where fp16 is not exact) + hub_reduce_kernel + "
                      "hub_rows_half_kernel + hub_scale_kernel, after the remainder's tf32_pack_kernel "
                      f"(column-scaled, slice maxima) + gather_kernel<Packed> over the {H.rest.phases}-phase "
                      "BCSR (row-scaled sums; all timed)")
            extra["path"] = (f"binary hybrid: 32-column steps of >= {BINARY_MIN_STEP_NNZ} entries as pattern tiles "
                             f"on the sparse MFMA "
                             f"over 2^e TF32(c X) (fp16 where exact, else bf16 halves) + packed gather of the "
                             f"remainder's pattern over its "
                             f"{H.rest.phases}-phase BCSR; A = diag(r) P diag(c) with the sym-norm scales")
        elif reuse >= PACK_MIN_REUSE:
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
    if args.config in (2, 3) and not args.profile_step:
        # SWTCF conversion of the same COO (S = 16), GEdges/s as the
        # reference's converter driver prints it (swtcf_convert_main.cu:417)
        m = swtcf.DeviceSWTCFMatrix(n, n, nnz, 16)
        ws = swtcf.SWTCFConvertWorkspace(nnz, n, 16)
        reps = 5 if args.config == 2 else 3
        conv_ms = timed(lambda: swtcf.convertCOOToSWTCF(r32, c32, nnz, m, ws), reps, 1)
        assert ws.device_error() == 0
        extra["convert_ms"] = round(conv_ms, 4)
        extra["convert_gedges_per_s"] = round(nnz / conv_ms / 1e6, 3)
        extra["convert_input_order"] = "(dst, src), as the generator lists the COO"
        # the same COO shuffled: every digit of the sort runs
        perm = torch.randperm(nnz, device="cuda", generator=torch.Generator(device="cuda").manual_seed(5))
        rs32, cs32 = r32[perm].contiguous(), c32[perm].contiguous()
        del perm
        conv_s = timed(lambda: swtcf.convertCOOToSWTCF(rs32, cs32, nnz, m, ws), reps, 1)
        assert ws.device_error() == 0
        extra["convert_shuffled_ms"] = round(conv_s, 4)
        extra["convert_shuffled_gedges_per_s"] = round(nnz / conv_s / 1e6, 3)
        del rs32, cs32
        if args.config in (2, 3):
            extra["swtcf"] = swtcf_plan_timings(torch, swtcf, m, n, nnz, args.config)
        del m, ws
        if args.config == 3:
            torch.cuda.empty_cache()
            extra["extension"] = extension_timings(torch, swtcf, r32, c32, n, F, X)
    if args.copy_calibration_mib:
        copy_calibration(args.copy_calibration_mib)
    if args.profile_step:
        print(f"[bench] profile-step: the step runs {args.warmup + args.steps} times", file=sys.stderr, flush=True)
    ms, median = timed_stats(step, args.steps, args.warmup)
    flops = 2.0 * nnz * F
    if args.config == 1:
        if not args.profile_step:
            # the kernel is shorter than a launch from Python: the same
            # launches replayed from a HIP graph give the GPU's time a product
            # (the reference times its launches from C++,
            # swtcf_spmm_main.cu:203-247)
            g_ms = graph_step_ms(torch, step, 100)
            extra["graph_ms_per_step"] = round(g_ms, 5)
            extra["graph_GFLOPs"] = round(flops / (g_ms * 1e-3) / 1e9, 3)
        torch.cuda.synchronize()
        Y.zero_()
        step()
    torch.cuda.synchronize()
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baselines(args, rows, cols, vals, X, n, Y, args.config, extra)
    # the traffic files hold the default path's kernels
    roof = roofline(flops, bytes_alg(n, n, nnz, F), ms, None if args.no_hybrid else traffic_of(args.config), kernel)
    config = {"workload": WORKLOADS[args.config], "n": n, "nnz": nnz, "F": F}
    return line_for(args, round(flops / (ms * 1e-3) / 1e9, 3), "GFLOP/s", ms, "fp32", config, roof, cpu, extra,
                    median=median)


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

    if args.copy_calibration_mib:
        copy_calibration(args.copy_calibration_mib)
    ms, median = timed_stats(step, args.steps, args.warmup)
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
    if not args.profile_step:
        extra["packed_rows"] = packed_rows_step(torch, table, X, cols, g1, F, Y, cold_rows_used, args)
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baselines(args, rows, cols, None, X, n, Y, 4, extra)
    # One launch (mixed_forward_kernel) interleaves the HBM-bound hot gather
    # with the scatter of cold rows read across the host link; the link bounds
    # it: the cold rows' bytes over PCIe Gen5 x16 (64 GB/s per direction).
    b_alg = bytes_alg(n, n, nnz, F)
    hbm_achieved = b_alg / (ms * 1e-3) / 1e9
    link_achieved = cold_bytes / (ms * 1e-3) / 1e9
    traffic = traffic_of(4)
    roof = {"bound": "host_link", "achieved": round(link_achieved, 2), "peak": PCIE_PEAK_GBPS, "unit": "GB/s",
            "frac": round(link_achieved / PCIE_PEAK_GBPS, 4),
            "traffic": None if traffic is None else traffic["hbm_bytes_per_launch"],
            "kernel": "mixed_forward_kernel (gather_body<Mixed> + scatter_body<Mixed>)",
            "bytes_alg_per_launch": cold_bytes,
            "hbm": {"achieved": round(hbm_achieved, 2), "peak": HBM_PEAK_GBPS,
                    "frac": round(hbm_achieved / HBM_PEAK_GBPS, 4), "bytes_alg_per_launch": b_alg}}
    config = {"workload": WORKLOADS[4], "n": n, "nnz": nnz, "F": F}
    table.free()
    return line_for(args, round(2.0 * nnz * F / (ms * 1e-3) / 1e9, 3), "GFLOP/s", ms, "fp32", config, roof,
                    cpu, extra, median=median)


def gcn_timings(args, torch, cfg):
    """Config 5: one full-graph GCN training epoch per step (at most 10 timed
    after 3), each layer's forward+backward alone, and the epoch over packed
    TF32 feature rows.  Returns (epoch ms, steps, warmup, extra)."""
    from tcc_amd import gcn

    n, F = cfg["n"], cfg["F"]
    hidden, classes = 256, 2
    rows, cols, X, table, g1, g2 = gcn_inputs(torch, cfg)
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
    if args.profile_step:
        print(f"[bench] profile-step: the epoch runs {warmup + steps} times", file=sys.stderr, flush=True)
    ms, median = timed_stats(epoch, steps, warmup)
    first_loss, last_loss = float(losses[0].item()), float(losses[-1].item())
    if args.profile_step:
        table.free()
        return ms, steps, warmup, {"loss_first": first_loss, "loss_last": last_loss}, rows.numel()

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
             "epoch_median_ms": round(median, 4),
             "layer_times": "each layer alone, through its own autograd function",
             "epoch_ms_packed_feature_rows": round(ms_packed, 4),
             "layer1_fwd_bwd_ms": round(l1, 4), "layer2_fwd_bwd_ms": round(l2, 4),
             "layer1": f"mixed SpMM F={F} (hot BCSR + cold BCSC) + GEMM {F}x{hidden}; backward dW GEMM",
             "layer2": f"A(XW): GEMM {hidden}x{classes}, BCSR SpMM F={classes}; backward A^T SpMM F={classes}, "
                       f"dW and dX GEMMs",
             "loss_first": first_loss, "loss_last": last_loss}
    table.free()
    return ms, steps, warmup, extra, rows.numel()


def bench_gcn(args, torch, swtcf, cfg):
    n, F = cfg["n"], cfg["F"]
    ms, steps, warmup, extra, nnz = gcn_timings(args, torch, cfg)
    config = {"workload": WORKLOADS[5], "n": n, "nnz": nnz, "F": F, "hidden": 256, "classes": 2}
    line = line_for(args, round(ms, 4), "ms", ms, "fp32", config, None, None, extra, higher=False,
                    median=extra.get("epoch_median_ms"))
    line["steps"], line["warmup"] = steps, warmup
    return line


def extra_configs(args, torch, swtcf):
    """Configs 1, 2 and 4's steps and config 5's epoch and layer times, for
    the config-3 line's `extra` (each with its own default step counts)."""
    from tcc_amd.graphs import CONFIGS

    out = {}
    a1 = copy.copy(args)
    a1.config, a1.steps, a1.warmup, a1.no_cpu_baseline, a1.copy_calibration_mib = 1, 500, 50, True, 0
    l1 = bench_spmm(a1, torch, swtcf, CONFIGS[1])
    out["config1"] = {"workload": WORKLOADS[1], "ms_per_step": l1["ms_per_step"], "GFLOPs": l1["value"],
                      "steps": 500, "warmup": 50, "roofline": l1["roofline"], "path": "launchSWTCFSpMM (S = 16)",
                      "convert_ms": l1["extra"].get("convert_ms"),
                      "convert_shuffled_ms": l1["extra"].get("convert_shuffled_ms"),
                      "graph_ms_per_step": l1["extra"].get("graph_ms_per_step"),
                      "graph_GFLOPs": l1["extra"].get("graph_GFLOPs")}
    torch.cuda.empty_cache()
    a2 = copy.copy(args)
    a2.config, a2.steps, a2.warmup, a2.no_cpu_baseline, a2.copy_calibration_mib = 2, 500, 50, True, 0
    l2 = bench_spmm(a2, torch, swtcf, CONFIGS[2])
    out["config2"] = {"workload": WORKLOADS[2], "ms_per_step": l2["ms_per_step"], "GFLOPs": l2["value"],
                      "steps": 500, "warmup": 50, "roofline": l2["roofline"], "path": l2["extra"].get("path"),
                      "convert_ms": l2["extra"].get("convert_ms"),
                      "convert_shuffled_ms": l2["extra"].get("convert_shuffled_ms"), "swtcf": l2["extra"].get("swtcf")}
    torch.cuda.empty_cache()
    a4 = copy.copy(args)
    a4.config, a4.steps, a4.warmup, a4.no_cpu_baseline, a4.copy_calibration_mib = 4, 20, 3, True, 0
    l4 = bench_mixed(a4, torch, swtcf, CONFIGS[4])
    out["config4"] = {"workload": WORKLOADS[4], "ms_per_step": l4["ms_per_step"], "GFLOPs": l4["value"],
                      "steps": 20, "warmup": 3, "roofline": l4["roofline"],
                      "packed_rows": l4["extra"].get("packed_rows")}
    torch.cuda.empty_cache()
    a5 = copy.copy(args)
    a5.config, a5.steps, a5.warmup = 5, 10, 3
    ms, steps, warmup, e5, _ = gcn_timings(a5, torch, CONFIGS[5])
    out["config5"] = {"workload": WORKLOADS[5], "epoch_ms": round(ms, 4), "epoch_median_ms": e5["epoch_median_ms"],
                      "steps": steps, "warmup": warmup,
                      "layer1_fwd_bwd_ms": e5["layer1_fwd_bwd_ms"], "layer2_fwd_bwd_ms": e5["layer2_fwd_bwd_ms"],
                      "epoch_ms_packed_feature_rows": e5["epoch_ms_packed_feature_rows"],
                      "loss_first": e5["loss_first"], "loss_last": e5["loss_last"], "epoch": e5["epoch"]}
    return out


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
    if args.profile_convert:
        print(json.dumps(bench_convert(args, torch, swtcf, cfg)), flush=True)
        return 0
    if args.swtcf_ab:
        print(json.dumps(bench_swtcf_ab(args, torch, swtcf)), flush=True)
        return 0
    if args.swtcf_int8:
        print(json.dumps(bench_swtcf_int8(args, torch, swtcf)), flush=True)
        return 0
    if args.atomic_probe_mib:
        print(json.dumps(atomic_probe(args, torch, swtcf)), flush=True)
        return 0
    if args.swtcf_step:
        if args.config not in (2, 3):
            raise SystemExit("--swtcf-step takes configs 2-3 (config 1's step is the SWTCF SpMM already)")
        if args.no_swtcf_plans:
            swtcf._lib.lib().tcc_swtcf_set_plans(0)
        print(json.dumps(bench_swtcf_step(args, torch, swtcf, cfg)), flush=True)
        return 0
    if args.config in (1, 2, 3):
        line = bench_spmm(args, torch, swtcf, cfg)
    elif args.config == 4:
        line = bench_mixed(args, torch, swtcf, cfg)
    else:
        line = bench_gcn(args, torch, swtcf, cfg)
    if args.config == 3 and not args.no_extra:
        torch.cuda.empty_cache()
        line["extra"].update(extra_configs(args, torch, swtcf))
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
