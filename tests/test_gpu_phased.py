"""Phased BCSR (tcc_coo_to_bcsr_phased): the matrix's column slices stacked
vertically, every window adding into window w % (windows / phases).

Checked against the ordinary build and the CSR oracle, through the C-ABI:
- the arrays: every window of phase p holds only columns of phase p
  (c * P // num_cols == p), and per output window the phases together hold
  exactly the ordinary BCSR's (column, row, value) entries;
- the products: bcsr_spmm (also F <= 16, the narrow kernel, whose windows
  then all add into a zeroed Y) and bcsr_spmm_packed, Y = AX and Y += AX, against the
  fp64 oracle on TF32-rounded inputs at rel-L2 <= 1e-5, as test_gpu_spmm;
- edge cases: no edges, fewer columns than phases, one phase;
- entry points that take no phased matrix return TCC_ERR_UNSUPPORTED.
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


def random_coo(nr, nc, nnz, seed, hubs):
    rng = np.random.default_rng(seed)
    nnz = max(0, min(nnz, nr * nc))
    if hubs:
        p_r = rng.pareto(1.2, nr) + 1e-3
        p_c = rng.pareto(1.2, nc) + 1e-3
        r = rng.choice(nr, size=2 * nnz + 1, p=p_r / p_r.sum())
        c = rng.choice(nc, size=2 * nnz + 1, p=p_c / p_c.sum())
        keys = np.unique(r.astype(np.int64) * nc + c)[:nnz]
    else:
        keys = np.sort(rng.choice(nr * nc, size=nnz, replace=False))
    return (keys // nc).astype(np.uint32), (keys % nc).astype(np.uint32)


def entries(h, windows_per_phase, phases):
    """(output window, column, row in window, value) of every stored entry."""
    out = []
    rwo = h["rowWindowOffset"]
    a2b = h["sparseA2B"].reshape(-1, 8)
    bits = h["tcLocalBit"]
    tco = h["tcOffset"]
    data = h["data"]
    for v in range(len(rwo) - 1):
        for b in range(rwo[v], rwo[v + 1]):
            rank = 0
            for bit in range(64):
                if (int(bits[b]) >> bit) & 1:
                    r, c = divmod(bit, 8)
                    val = data[tco[b] + rank] if data is not None else 1.0
                    out.append((v % windows_per_phase, int(a2b[b, c]), r, float(val), v // windows_per_phase))
                    rank += 1
    return out


@pytest.mark.parametrize("phases", [2, 3, 8])
def test_phased_arrays_match_ordinary_build(phases):
    from tcc_amd import swtcf

    nr, nc = 300, 700
    dst, src = random_coo(nr, nc, 6000, 11 + phases, hubs=True)
    vals = torch.from_numpy(np.random.default_rng(3).uniform(-1, 1, dst.size).astype(np.float32)).cuda()
    A = swtcf.coo_to_bcsr(dev_u32(dst), dev_u32(src), vals, nr, nc)
    Ap = swtcf.coo_to_bcsr(dev_u32(dst), dev_u32(src), vals, nr, nc, phases=phases)
    W = (nr + 7) // 8
    assert Ap.phases == phases and Ap.num_windows == phases * W and Ap.out_windows == W
    assert Ap.view.num_rows == nr and Ap.view.nnz == dst.size
    h, hp = A.to_host(), Ap.to_host()
    assert hp["phases"] == phases
    e = entries(h, W, 1)
    ep = entries(hp, W, phases)
    assert len(ep) == dst.size
    for (w, c, r, v, p) in ep:
        assert c * phases // nc == p, "a column in the wrong phase"
    key = lambda t: (t[0], t[1], t[2])
    assert sorted((key(t), t[3]) for t in e) == sorted((key(t), t[3]) for t in ep)
    # within each window, columns ascend and padding only ends a window
    rwo = hp["rowWindowOffset"]
    a2b = hp["sparseA2B"].reshape(-1, 8)
    for v in range(len(rwo) - 1):
        cols = a2b[rwo[v]:rwo[v + 1]].ravel()
        valid = cols[cols != 0xFFFFFFFF]
        assert np.all(np.diff(valid.astype(np.int64)) > 0)
        assert np.all(cols[valid.size:] == 0xFFFFFFFF)


CASES = [
    # nr, nc, nnz, F, phases, hubs, values, unit blocks
    (1000, 1300, 20000, 128, 4, True, True, 0),
    (777, 2049, 30000, 602, 4, True, True, 3),
    (640, 500, 9000, 300, 3, False, False, 16),
    (1201, 900, 40000, 64, 8, True, True, 5),
    (333, 3, 700, 32, 8, False, True, 0),  # fewer columns than phases
    (2048, 2048, 15000, 5, 4, True, True, 0),  # F <= 16: the narrow kernel
    (3000, 2500, 40000, 2, 8, True, True, 0),  # F = 2, as a GCN's last layer
    (1100, 1700, 30000, 16, 3, True, False, 9),  # F = 16, units cutting windows
    (900, 1100, 12000, 1, 2, False, True, 7),
    (1500, 1500, 25000, 256, 16, True, False, 2),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_phased_products(gpu, oracle, case):
    from tcc_amd import swtcf

    nr, nc, nnz, F, phases, hubs, values, K = CASES[case]
    print(f"case {case}: nr={nr} nc={nc} nnz={nnz} F={F} phases={phases} K={K}", flush=True)
    dst, src = random_coo(nr, nc, nnz, 500 + case, hubs)
    rng = np.random.default_rng(600 + case)
    vals = rng.uniform(-1, 1, dst.size).astype(np.float32) if values else None
    X = rng.standard_normal((nc, F)).astype(np.float32)
    order = np.lexsort((src, dst))
    rowptr = np.zeros(nr + 1, np.int64)
    rowptr[1:] = np.cumsum(np.bincount(dst, minlength=nr))
    want = oracle.csr_spmm(rowptr, src[order], None if vals is None else vals[order], X, use_tf32=True)

    tv = None if vals is None else torch.from_numpy(vals).cuda()
    A = swtcf.coo_to_bcsr(dev_u32(dst), dev_u32(src), tv, nr, nc, phases=phases).set_unit_blocks(K)
    rows8 = A.out_windows * 8
    Xd = torch.from_numpy(X).cuda()
    Y = swtcf.bcsr_spmm(A, Xd, torch.full((rows8, F), 5.0, device="cuda")).cpu().numpy()
    assert rel_l2(Y[:nr], want) <= REL, "bcsr"
    assert np.all(Y[nr:] == 0)

    P = swtcf.tf32_pack(Xd)
    Yp = swtcf.bcsr_spmm_packed(A, P, F, torch.full((rows8, F), 5.0, device="cuda")).cpu().numpy()
    assert rel_l2(Yp[:nr], want) <= REL, "packed"

    Y0 = rng.standard_normal((rows8, F)).astype(np.float32)
    Ya = swtcf.bcsr_spmm(A, Xd, torch.from_numpy(Y0.copy()).cuda(), accumulate=True).cpu().numpy()
    assert rel_l2(Ya[:nr], Y0[:nr].astype(np.float64) + want) <= REL, "bcsr accumulate"
    Ypa = swtcf.bcsr_spmm_packed(A, P, F, torch.from_numpy(Y0.copy()).cuda(), accumulate=True).cpu().numpy()
    assert rel_l2(Ypa[:nr], Y0[:nr].astype(np.float64) + want) <= REL, "packed accumulate"


def test_phased_without_edges():
    from tcc_amd import swtcf

    e = torch.empty(0, dtype=torch.int32, device="cuda")
    A = swtcf.coo_to_bcsr(e, e, None, 50, 40, phases=4)
    assert A.view.num_TCBlocks == 0 and A.num_windows == 4 * 7 and A.out_windows == 7
    Y = swtcf.bcsr_spmm(A, torch.randn(40, 64, device="cuda"), torch.full((56, 64), 3.0, device="cuda"))
    assert torch.count_nonzero(Y).item() == 0


def test_phases_one_is_the_ordinary_build():
    from tcc_amd import swtcf

    dst, src = random_coo(400, 500, 5000, 21, hubs=True)
    A = swtcf.coo_to_bcsr(dev_u32(dst), dev_u32(src), None, 400, 500)
    A1 = swtcf.coo_to_bcsr(dev_u32(dst), dev_u32(src), None, 400, 500, phases=1)
    h, h1 = A.to_host(), A1.to_host()
    for k in ("rowWindowOffset", "tcOffset", "sparseA2B", "tcLocalBit"):
        assert np.array_equal(h[k], h1[k]), k
    assert h1["phases"] == 1


def test_phased_rejected_where_unsupported():
    from tcc_amd import swtcf
    from tcc_amd._lib import TccError
    from tcc_amd.hostmem import PinnedArray

    nr = nc = 256
    F = 16
    dst, src = random_coo(nr, nc, 3000, 31, hubs=False)
    A = swtcf.coo_to_bcsr(dev_u32(dst), dev_u32(src), None, nr, nc, phases=2)
    B = swtcf.coo_to_bcsc(dev_u32(dst), dev_u32(src), None, nr, nc)
    hot = torch.zeros(nc, F, device="cuda")
    cpu = PinnedArray((nc, F))
    ptrs = torch.tensor([hot.data_ptr()], dtype=torch.int64, device="cuda")
    ident = torch.arange(nc, dtype=torch.int32, device="cuda")
    srcd = swtcf.feature_source(ident, ident, ptrs, nc, cpu.device_ptr, nc * F)
    C = torch.empty((A.out_windows + 1) * 8, F, device="cuda")
    with pytest.raises(TccError):
        swtcf.spmm_cnic_forward_mixed(A, B, srcd, C, F)
    with pytest.raises(TccError):
        swtcf.bcsr_spmm_mixed(A, srcd, torch.empty(A.out_windows * 8, F, device="cuda"), F)
    cpu.free()
