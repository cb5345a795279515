"""Seeded random shapes for every block-SpMM entry point against the CSR
oracle, through the C-ABI.

Each case draws row and column counts that need not be multiples of 8, F
from 1 to 700 (the narrow gather, V = 1/2/4 chunk gathers and packed rows
of one to three chunks), densities from a handful of edges to ~20%, uniform
or R-MAT (hub) structure, values or none, and unit sizes that cut windows
between waves.  Tolerance as in test_gpu_spmm: rel-L2 <= 1e-5 against the
fp64 oracle on TF32-rounded inputs (the A^T product in plain fp32); a wrong
row, column, value rank or unit boundary gives errors of order 1.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

REL = 1e-5


def rel_l2(y, ref):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(y - ref) / (den if den > 0 else 1.0))


def dev_u32(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).cuda()


def make_case(i):
    rng = np.random.default_rng(9000 + i)
    nr = int(rng.integers(1, 2500))
    nc = int(rng.integers(1, 2500))
    F = int(rng.choice([1, 2, 3, 5, 8, 13, 16, 17, 31, 64, 100, 128, 129, 200, 256, 257, 301, 512, 602, 700]))
    dens = float(rng.choice([1e-4, 1e-3, 5e-3, 0.02, 0.2]))
    nnz = max(1, min(nr * nc, int(nr * nc * dens)))
    if rng.random() < 0.5:  # uniform
        keys = np.sort(rng.choice(nr * nc, size=nnz, replace=False))
    else:  # R-MAT-like: hub rows and columns by skewed sampling
        p_r = rng.pareto(1.2, nr) + 1e-3
        p_c = rng.pareto(1.2, nc) + 1e-3
        r = rng.choice(nr, size=2 * nnz, p=p_r / p_r.sum())
        c = rng.choice(nc, size=2 * nnz, p=p_c / p_c.sum())
        keys = np.unique(r.astype(np.int64) * nc + c)[:nnz]
    dst = (keys // nc).astype(np.uint32)
    src = (keys % nc).astype(np.uint32)
    values = bool(rng.random() < 0.6)
    vals = rng.uniform(-1, 1, dst.size).astype(np.float32) if values else None
    K = int(rng.choice([0, 1, 2, 5, 16]))
    return dict(nr=nr, nc=nc, F=F, dst=dst, src=src, vals=vals, K=K, seed=9000 + i)


CASES = list(range(16))


@pytest.mark.parametrize("i", CASES)
def test_random_shape_all_products(gpu, oracle, i):
    from tcc_amd import swtcf

    c = make_case(i)
    nr, nc, F, dst, src, vals, K = c["nr"], c["nc"], c["F"], c["dst"], c["src"], c["vals"], c["K"]
    print(f"case {i}: nr={nr} nc={nc} F={F} nnz={dst.size} values={vals is not None} K={K}", flush=True)
    rng = np.random.default_rng(c["seed"] + 1)
    X = rng.standard_normal((nc, F)).astype(np.float32)
    order = np.lexsort((src, dst))
    rowptr = np.zeros(nr + 1, np.int64)
    rowptr[1:] = np.cumsum(np.bincount(dst, minlength=nr))
    v = None if vals is None else vals[order]
    want = oracle.csr_spmm(rowptr, src[order], v, X, use_tf32=True)
    tv = None if vals is None else torch.from_numpy(vals).cuda()
    Xd = torch.from_numpy(X).cuda()

    A = swtcf.coo_to_bcsr(dev_u32(dst), dev_u32(src), tv, nr, nc).set_unit_blocks(K)
    rows8 = A.view.num_rowWindows * 8
    Y = swtcf.bcsr_spmm(A, Xd, torch.full((rows8, F), 5.0, device="cuda")).cpu().numpy()
    assert rel_l2(Y[:nr], want) <= REL, "bcsr"
    assert np.all(Y[nr:] == 0)

    P = swtcf.tf32_pack(Xd)
    Yp = swtcf.bcsr_spmm_packed(A, P, F, torch.full((rows8, F), 5.0, device="cuda")).cpu().numpy()
    assert rel_l2(Yp[:nr], want) <= REL, "packed"

    B = swtcf.coo_to_bcsc(dev_u32(dst), dev_u32(src), tv, nr, nc).set_unit_blocks(K)
    Y0 = rng.standard_normal((nr, F)).astype(np.float32)
    Yc = torch.from_numpy(Y0.copy()).cuda()
    swtcf.bcsc_spmm(B, Xd, Yc)
    assert rel_l2(Yc.cpu().numpy(), Y0.astype(np.float64) + want) <= REL, "bcsc"

    dY = rng.standard_normal((nr, F)).astype(np.float32)
    corder = np.lexsort((dst, src))
    colptr = np.zeros(nc + 1, np.int64)
    colptr[1:] = np.cumsum(np.bincount(src, minlength=nc))
    wantT = oracle.csr_spmm(colptr, dst[corder], None if vals is None else vals[corder], dY, use_tf32=False)
    dX = swtcf.bcsc_transpose_spmm(B, torch.from_numpy(dY).cuda()).cpu().numpy()
    assert rel_l2(dX[:nc], wantT) <= REL, "transpose"
    assert np.all(dX[nc:] == 0)
