"""Row super-window BCSR (tcc_coo_to_sw_bcsr, tcc_sw_bcsr_spmm_packed).

Checked through the C-ABI:
- the arrays, exactly, against an independent numpy construction of the
  layout the header states (rows by degree descending then id, 64 per
  super-window; each super-window's columns by degree rank; 64-bit row
  masks; values pair by pair in mask-bit order; units of unit_pairs pairs);
- the products against the fp64 CSR oracle on TF32-rounded inputs
  (rel-L2 <= 1e-5, as the other gathers), Y = AX and Y += AX, over row
  counts off multiples of 64, empty rows, hub rows and hub columns, F from 1
  to 700 (a partial last chunk, chunks of one lane), values or none, and
  units from 1 pair (every super-window shared, atomics) to whole
  super-windows (direct stores);
- no edges, duplicate edges and out-of-range indices.
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
    keys = keys[np.random.default_rng(seed + 1).permutation(keys.size)]  # any COO order
    return (keys // nc).astype(np.uint32), (keys % nc).astype(np.uint32)


def reference_layout(dst, src, vals, nr, nc, unit_pairs, phases=1):
    """The layout of include/tcc_spmm_cnic.h (tcc_sw_bcsr), built with numpy."""
    dst = dst.astype(np.int64)
    src = src.astype(np.int64)
    rd = np.bincount(dst, minlength=nr)
    cd = np.bincount(src, minlength=nc)
    row_order = np.lexsort((np.arange(nr), -rd))
    rrank = np.empty(nr, np.int64)
    rrank[row_order] = np.arange(nr)
    crank = np.empty(nc, np.int64)
    crank[np.lexsort((np.arange(nc), -cd))] = np.arange(nc)
    G = (nr + 63) // 64
    ro = np.full(64 * G, 0xFFFFFFFF, np.uint32)
    ro[:nr] = row_order
    rr = rrank[dst]
    g, slot, cr = rr // 64, rr % 64, crank[src]
    order = np.lexsort((slot, cr, g))
    g, slot, cr, src_s = g[order], slot[order], cr[order], src[order]
    head = np.ones(order.size, bool)
    if order.size:
        head[1:] = (g[1:] != g[:-1]) | (cr[1:] != cr[:-1])
    pid = np.cumsum(head) - 1
    P = int(head.sum())
    mask = np.zeros(P, np.uint64)
    np.bitwise_or.at(mask, pid, (np.uint64(1) << slot.astype(np.uint64)))
    pair_col = src_s[head].astype(np.uint32)
    pair_value = np.nonzero(head)[0].astype(np.uint32)
    pair_group = g[head]
    group_offset = np.searchsorted(pair_group, np.arange(G + 1)).astype(np.uint32)
    # phase k >= 1 starts at the first column rank with >= ceil(k P / phases)
    # pairs of lower rank
    pair_rank = cr[head]
    cum_excl = np.concatenate([[0], np.cumsum(np.bincount(pair_rank, minlength=nc))[:-1]])
    bounds = [nc] * phases
    for k in range(1, phases):
        t = -(-k * P // phases)
        r = int(np.searchsorted(cum_excl, t, side="left")) if t > 0 else nc
        if r < nc:
            bounds[k] = r
    pair_phase = np.zeros(P, np.int64)
    for k in range(1, phases):
        pair_phase += pair_rank >= bounds[k]
    counts = np.zeros((phases, G), np.int64)
    np.add.at(counts, (pair_phase, pair_group), 1)
    units = []
    for ph in range(phases):
        for gg in range(G):
            start = int(group_offset[gg]) + int(counts[:ph, gg].sum())
            end = start + int(counts[ph, gg])
            n_units = -(-int(counts[ph, gg]) // unit_pairs)
            if ph == 0 and group_offset[gg + 1] == group_offset[gg]:
                n_units = 1
            for k in range(n_units):
                units.append((gg, start + k * unit_pairs, min(start + (k + 1) * unit_pairs, end)))
    data = None if vals is None else vals[order].astype(np.float32)
    return dict(rowOrder=ro, groupOffset=group_offset, pairCol=pair_col, pairMask=mask, pairValue=pair_value,
                data=data, units=np.array(units, np.uint32).reshape(-1, 3), num_pairs=P)


def oracle_product(oracle, dst, src, vals, nr, X):
    order = np.lexsort((src, dst))
    rowptr = np.zeros(nr + 1, np.int64)
    np.cumsum(np.bincount(dst.astype(np.int64), minlength=nr), out=rowptr[1:])
    return oracle.csr_spmm(rowptr, src[order], None if vals is None else vals[order], X, use_tf32=True)


@pytest.mark.parametrize("nr, nc, nnz, hubs, unit_pairs, values, phases", [
    (300, 700, 6000, True, 0, True, 1),
    (300, 700, 6000, True, 7, False, 1),
    (300, 700, 6000, True, 50, True, 4),
    (1, 50, 20, False, 0, True, 1),
    (1, 50, 20, False, 3, True, 16),
    (65, 9, 200, False, 3, True, 2),
    (1000, 400, 30000, True, 64, True, 3),
    (40, 30, 0, False, 0, False, 4),
])
def test_arrays_match_numpy_layout(gpu, nr, nc, nnz, hubs, unit_pairs, values, phases):
    from tcc_amd import swtcf

    dst, src = random_coo(nr, nc, nnz, nr + nc + nnz, hubs)
    vals = np.random.default_rng(5).uniform(-1, 1, dst.size).astype(np.float32) if values else None
    A = swtcf.coo_to_sw_bcsr(dev_u32(dst), dev_u32(src), None if vals is None else torch.from_numpy(vals).cuda(),
                             nr, nc, unit_pairs=unit_pairs, phases=phases)
    h = A.to_host()
    want = reference_layout(dst, src, vals, nr, nc, unit_pairs or 2048, phases)
    assert h["num_phases"] == phases
    assert h["num_pairs"] == want["num_pairs"] and h["num_groups"] == (nr + 63) // 64
    assert h["unit_pairs"] == (unit_pairs or 2048) and h["nnz"] == dst.size
    for k in ("rowOrder", "groupOffset", "pairCol", "pairMask", "units"):
        assert np.array_equal(h[k], want[k]), k
    if values:
        assert np.array_equal(h["pairValue"], want["pairValue"])
        assert np.array_equal(h["data"], want["data"])
    else:
        assert h["data"] is None


CASES = [
    # nr, nc, nnz, hubs, unit_pairs, values, F, phases
    (300, 700, 6000, True, 0, True, 602, 1),
    (300, 700, 6000, True, 0, True, 602, 4),
    (300, 700, 6000, True, 1, True, 90, 1),
    (300, 700, 6000, True, 33, False, 256, 3),
    (1000, 400, 30000, True, 64, True, 257, 1),
    (1000, 400, 30000, True, 0, False, 128, 8),
    (777, 1500, 20000, False, 31, True, 700, 2),
    (64, 64, 4096, False, 0, True, 64, 1),       # dense: every mask full
    (64, 64, 4096, False, 0, True, 64, 16),
    (200, 3000, 8000, True, 100, True, 1, 1),
    (200, 3000, 8000, True, 5, True, 3, 4),
    (129, 17, 300, False, 2, False, 5, 1),
    (5000, 5000, 60000, True, 0, True, 346, 4),
    (50, 200, 0, False, 0, True, 64, 4),         # no edges: zeros
]


@pytest.mark.parametrize("nr, nc, nnz, hubs, unit_pairs, values, F, phases", CASES)
def test_spmm_vs_oracle(gpu, oracle, nr, nc, nnz, hubs, unit_pairs, values, F, phases):
    from tcc_amd import swtcf

    print(f"sw_bcsr nr={nr} nc={nc} nnz={nnz} hubs={hubs} unit_pairs={unit_pairs} values={values} F={F} "
          f"phases={phases}", flush=True)
    dst, src = random_coo(nr, nc, nnz, 7 * nr + nc + F, hubs)
    rng = np.random.default_rng(F + nnz)
    vals = rng.uniform(-1, 1, dst.size).astype(np.float32) if values else None
    X = rng.standard_normal((nc, F)).astype(np.float32)
    A = swtcf.coo_to_sw_bcsr(dev_u32(dst), dev_u32(src), None if vals is None else torch.from_numpy(vals).cuda(),
                             nr, nc, unit_pairs=unit_pairs, phases=phases)
    P = swtcf.tf32_pack(torch.from_numpy(X).cuda())
    Y = swtcf.sw_bcsr_spmm_packed(A, P, F)
    want = oracle_product(oracle, dst, src, vals, nr, X)
    got = Y.cpu().numpy()
    assert got.shape == (nr, F)
    e = rel_l2(got, want)
    assert e <= REL, f"rel-L2 {e}"
    if nnz == 0:
        assert not np.any(got)
    # Y += A X on top of a nonzero Y
    Y0 = rng.standard_normal((nr, F)).astype(np.float32)
    Yd = torch.from_numpy(Y0).cuda()
    swtcf.sw_bcsr_spmm_packed(A, P, F, Yd, accumulate=True)
    e = rel_l2(Yd.cpu().numpy(), want + Y0)
    assert e <= REL, f"accumulate rel-L2 {e}"


def test_spmm_twice_same_buffers(gpu, oracle):
    """A second product into the same Y gives the same result (shared
    super-windows are zeroed again, not added to the previous Y)."""
    from tcc_amd import swtcf

    nr, nc, F = 500, 900, 300
    dst, src = random_coo(nr, nc, 15000, 3, True)
    X = np.random.default_rng(1).standard_normal((nc, F)).astype(np.float32)
    A = swtcf.coo_to_sw_bcsr(dev_u32(dst), dev_u32(src), None, nr, nc, unit_pairs=16, phases=4)
    P = swtcf.tf32_pack(torch.from_numpy(X).cuda())
    Y = swtcf.sw_bcsr_spmm_packed(A, P, F)
    first = Y.clone()
    swtcf.sw_bcsr_spmm_packed(A, P, F, Y)
    assert rel_l2(Y.cpu().numpy(), first.cpu().numpy()) <= 1e-6
    assert rel_l2(first.cpu().numpy(), oracle_product(oracle, dst, src, None, nr, X)) <= REL


def test_errors(gpu):
    from tcc_amd import _lib, swtcf

    dst = np.array([0, 1, 1], np.uint32)
    src = np.array([2, 3, 3], np.uint32)
    with pytest.raises(_lib.TccError, match="duplicate"):
        swtcf.coo_to_sw_bcsr(dev_u32(dst), dev_u32(src), None, 4, 4)
    with pytest.raises(_lib.TccError, match="out of range"):
        swtcf.coo_to_sw_bcsr(dev_u32(np.array([0, 9], np.uint32)), dev_u32(np.array([0, 1], np.uint32)), None, 4, 4)
    with pytest.raises(_lib.TccError, match="out of range"):
        swtcf.coo_to_sw_bcsr(dev_u32(np.array([0, 1], np.uint32)), dev_u32(np.array([0, 4], np.uint32)), None, 4, 4)
    with pytest.raises(_lib.TccError, match="16 phases"):
        swtcf.coo_to_sw_bcsr(dev_u32(np.array([0], np.uint32)), dev_u32(np.array([1], np.uint32)), None, 4, 4,
                             phases=17)
    A = swtcf.coo_to_sw_bcsr(dev_u32(np.array([0], np.uint32)), dev_u32(np.array([1], np.uint32)), None, 4, 4)
    buf = torch.empty(64, dtype=torch.uint8, device="cuda")
    with pytest.raises(_lib.TccError, match="aligned"):
        swtcf.sw_bcsr_spmm_packed(A, buf[1:], 4)
