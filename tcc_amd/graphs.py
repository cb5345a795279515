"""Seeded synthetic graphs and features for the benchmark configurations.

The reference ships no input graphs (its CLIs read raw u32 COO files,
src/swtcf_convert_main.cu:16-30); these generators produce the inputs the
benchmark configurations describe.  Edges are (dst, src) = (row, col) of A.

* uniform_graph: every row gets `deg` distinct columns drawn uniformly.
* rmat_graph:    R-MAT with quadrant probabilities (a, b, c, 1-a-b-c) over
                 scale = ceil(log2 n) levels, ids >= n rejected, one seeded
                 vertex permutation applied to rows and columns, duplicates
                 removed, regenerated until exactly `nnz` distinct edges.

Generation runs with torch on the given device; a fixed seed gives the same
graph on every run on the same kind of device.
"""
from __future__ import annotations

import math

import numpy as np
import torch


def uniform_graph(n: int, deg: int, seed: int, device="cpu"):
    """Rows 0..n-1 with `deg` distinct uniform columns each (config 1)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    # argsort of random keys = a uniform random subset without replacement
    cols = torch.empty((n, deg), dtype=torch.int64)
    chunk = max(1, (1 << 22) // max(n, 1))
    for r0 in range(0, n, chunk):
        r1 = min(n, r0 + chunk)
        keys = torch.rand((r1 - r0, n), generator=g)
        cols[r0:r1] = torch.topk(keys, deg, dim=1).indices
    rows = torch.arange(n, dtype=torch.int64).repeat_interleave(deg)
    cols = cols.reshape(-1)
    order = torch.argsort(rows * n + cols)
    return rows[order].to(device), cols[order].to(device)


def rmat_graph(n: int, nnz: int, seed: int, a=0.57, b=0.19, c=0.19, device="cpu"):
    """R-MAT edges sorted by (row, col); returns int64 (rows, cols) on `device`."""
    dev = torch.device(device)
    gen = torch.Generator(device=dev).manual_seed(seed)
    scale = max(1, math.ceil(math.log2(n)))
    perm = torch.randperm(n, generator=gen, device=dev)
    keys = torch.empty(0, dtype=torch.int64, device=dev)
    rounds = 0
    while keys.numel() < nnz:
        need = nnz - keys.numel()
        m = int(need * 1.2) + 4096
        r = torch.zeros(m, dtype=torch.int64, device=dev)
        cc = torch.zeros(m, dtype=torch.int64, device=dev)
        for lvl in range(scale):
            u = torch.rand(m, generator=gen, device=dev)
            rb = u >= (a + b)
            cb = ((u >= a) & (u < a + b)) | (u >= a + b + c)
            r |= rb.to(torch.int64) << lvl
            cc |= cb.to(torch.int64) << lvl
        ok = (r < n) & (cc < n)
        k = perm[r[ok]] * n + perm[cc[ok]]
        keys = torch.unique(torch.cat([keys, k]))
        rounds += 1
        if rounds > 64:
            raise RuntimeError("R-MAT generation did not reach the requested nnz")
    if keys.numel() > nnz:
        sel = torch.randperm(keys.numel(), generator=gen, device=dev)[:nnz]
        keys = torch.sort(keys[sel]).values
    return keys // n, keys % n


def sym_norm_values(rows: torch.Tensor, cols: torch.Tensor, n: int) -> torch.Tensor:
    """v_ij = 1 / sqrt(rowdeg_i * coldeg_j) in fp32."""
    rd = torch.bincount(rows, minlength=n).to(torch.float64)
    cd = torch.bincount(cols, minlength=n).to(torch.float64)
    return (1.0 / torch.sqrt(rd[rows] * cd[cols])).to(torch.float32)


def sym_norm_scales(rows: torch.Tensor, cols: torch.Tensor, n: int):
    """(r, c) fp32 with r_i = rowdeg_i^-1/2, c_j = coldeg_j^-1/2 (0 for an
    empty row or column): sym_norm_values' v_ij = r_i c_j as row and column
    scales (each fp32 product within 2 ulp of v_ij)."""
    rd = torch.bincount(rows, minlength=n).to(torch.float64)
    cd = torch.bincount(cols, minlength=n).to(torch.float64)
    r = torch.where(rd > 0, 1.0 / torch.sqrt(rd.clamp_min(1.0)), torch.zeros_like(rd))
    c = torch.where(cd > 0, 1.0 / torch.sqrt(cd.clamp_min(1.0)), torch.zeros_like(cd))
    return r.to(torch.float32), c.to(torch.float32)


def to_csr_numpy(rows: torch.Tensor, cols: torch.Tensor, n_rows: int, vals: torch.Tensor | None = None):
    """(rowptr int64, colind uint32, vals float32|None) of edges sorted by (row, col)."""
    r = rows.cpu().numpy().astype(np.int64)
    c = cols.cpu().numpy().astype(np.int64)
    key = r * (int(c.max()) + 1 if c.size else 1) + c
    order = np.arange(r.size) if bool(np.all(key[1:] >= key[:-1])) else np.lexsort((c, r))
    rowptr = np.zeros(n_rows + 1, np.int64)
    np.cumsum(np.bincount(r, minlength=n_rows), out=rowptr[1:])
    v = None if vals is None else vals.cpu().numpy().astype(np.float32)[order]
    return rowptr, c[order].astype(np.uint32), v


CONFIGS = {
    1: dict(kind="uniform", n=4096, deg=16, F=32, seed=1, values=False),
    2: dict(kind="rmat", n=169_000, nnz=1_170_000, F=128, seed=2, values=True),
    3: dict(kind="rmat", n=233_000, nnz=114_000_000, F=602, seed=3, values=True),
    4: dict(kind="rmat", n=2_450_000, nnz=61_900_000, F=100, seed=4, values=False),
    5: dict(kind="rmat", n=2_450_000, nnz=61_900_000, F=100, seed=4, values=False),
}


def make_graph(cfg: int, device="cpu"):
    c = CONFIGS[cfg]
    if c["kind"] == "uniform":
        rows, cols = uniform_graph(c["n"], c["deg"], c["seed"], device=device)
    else:
        rows, cols = rmat_graph(c["n"], c["nnz"], c["seed"], device=device)
    vals = sym_norm_values(rows, cols, c["n"]) if c["values"] else None
    return rows, cols, vals


def make_features(n: int, F: int, seed: int, dist: str = "normal", device="cpu") -> torch.Tensor:
    g = torch.Generator(device=torch.device(device)).manual_seed(seed + 1000)
    if dist == "uniform":
        return (torch.rand((n, F), generator=g, device=device) * 2.0 - 1.0).contiguous()
    return torch.randn((n, F), generator=g, device=device).contiguous()
