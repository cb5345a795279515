"""Dense hub tiles + sparse remainder (tcc_coo_to_hybrid, tcc_hybrid_spmm).

Checked through the C-ABI:
- the arrays, exactly, against an independent numpy construction of the
  layout include/tcc_spmm_cnic.h states: rows and columns ranked by degree
  (descending, then index); 16x16 tiles of the reordered matrix with at
  least min_tile_nnz entries, sorted by (row block, column block); values
  TF32-rounded at A(row l%16, column 4s + l/16) -> tileVals[t][l][s]; units
  of unit_tiles tiles; the other entries' BCSR equal to the oracle's BCSR of
  exactly those entries;
- the products against the fp64 CSR oracle on TF32-rounded inputs (rel-L2
  <= 1e-5), Y = AX and Y += AX, over thresholds from 1 (every tile dense) to
  256 (no tile dense), row blocks shared by up to hundreds of units (their
  partial sums reduced in a second pass), unit sizes 1 to 64, phased
  remainders, F from 1 to 700, values or none, hubs or uniform;
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
        p_r = rng.pareto(1.0, nr) + 1e-3
        p_c = rng.pareto(1.0, nc) + 1e-3
        r = rng.choice(nr, size=3 * nnz + 1, p=p_r / p_r.sum())
        c = rng.choice(nc, size=3 * nnz + 1, p=p_c / p_c.sum())
        keys = np.unique(r.astype(np.int64) * nc + c)[:nnz]
    else:
        keys = np.sort(rng.choice(nr * nc, size=nnz, replace=False))
    keys = keys[np.random.default_rng(seed + 1).permutation(keys.size)]
    return (keys // nc).astype(np.uint32), (keys % nc).astype(np.uint32)


def tf32(a):
    b = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
    fin = (b & 0x7F800000) != 0x7F800000
    return np.where(fin, (b + 0x1000) & 0xFFFFE000, b).astype(np.uint32).view(np.float32)


def reference_layout(dst, src, vals, nr, nc, min_nnz, unit_tiles):
    dst = dst.astype(np.int64)
    src = src.astype(np.int64)
    rorder = np.lexsort((np.arange(nr), -np.bincount(dst, minlength=nr)))
    corder = np.lexsort((np.arange(nc), -np.bincount(src, minlength=nc)))
    rrank = np.empty(nr, np.int64)
    rrank[rorder] = np.arange(nr)
    crank = np.empty(nc, np.int64)
    crank[corder] = np.arange(nc)
    RB, CB = (nr + 15) // 16, (nc + 15) // 16
    row_order = np.full(16 * RB, 0xFFFFFFFF, np.uint32)
    row_order[:nr] = rorder
    rr, cr = rrank[dst], crank[src]
    tile = (rr // 16) * CB + cr // 16
    keys, counts = np.unique(tile, return_counts=True)
    dense_keys = keys[counts >= min_nnz]
    in_dense = np.isin(tile, dense_keys)
    tid = np.searchsorted(dense_keys, tile[in_dense])
    vals_all = np.ones(dst.size, np.float32) if vals is None else vals
    tv = np.zeros((dense_keys.size, 64, 4), np.float32)
    i, j = rr[in_dense] % 16, cr[in_dense] % 16
    tv[tid, i + 16 * (j % 4), j // 4] = tf32(vals_all[in_dense])
    rb, cb = dense_keys // CB, dense_keys % CB
    rbo = np.searchsorted(rb, np.arange(RB + 1)).astype(np.uint32)
    units = []
    for b in range(RB):
        t0, t1 = int(rbo[b]), int(rbo[b + 1])
        for k in range(-(-(t1 - t0) // unit_tiles)):
            units.append((b, t0 + k * unit_tiles, min(t0 + (k + 1) * unit_tiles, t1)))
    hub_cols = min(16 * (int(cb.max()) + 1), nc) if cb.size else 0
    return dict(rowOrder=row_order, hubColOrder=corder[:hub_cols].astype(np.uint32), rowBlockOffset=rbo,
                tileCol=cb.astype(np.uint32), tileVals=tv, units=np.array(units, np.uint32).reshape(-1, 3),
                hub_cols=hub_cols, rest=~in_dense)


def oracle_product(oracle, dst, src, vals, nr, X):
    order = np.lexsort((src, dst))
    rowptr = np.zeros(nr + 1, np.int64)
    np.cumsum(np.bincount(dst.astype(np.int64), minlength=nr), out=rowptr[1:])
    return oracle.csr_spmm(rowptr, src[order], None if vals is None else vals[order], X, use_tf32=True)


@pytest.mark.parametrize("nr, nc, nnz, hubs, min_nnz, unit_tiles, values", [
    (500, 700, 30000, True, 32, 4, True),
    (500, 700, 30000, True, 8, 0, False),
    (129, 33, 2000, False, 1, 3, True),      # every occupied tile dense
    (300, 300, 5000, True, 256, 0, True),    # no tile dense: all in the remainder
    (17, 1000, 3000, True, 20, 1, True),
    (60, 60, 0, False, 32, 0, True),
])
def test_arrays_match_numpy_layout(gpu, oracle, nr, nc, nnz, hubs, min_nnz, unit_tiles, values):
    from tcc_amd import swtcf

    dst, src = random_coo(nr, nc, nnz, nr * 3 + nc + nnz, hubs)
    vals = np.random.default_rng(9).uniform(-1, 1, dst.size).astype(np.float32) if values else None
    H = swtcf.coo_to_hybrid(dev_u32(dst), dev_u32(src), None if vals is None else torch.from_numpy(vals).cuda(), nr, nc,
                            min_tile_nnz=min_nnz, unit_tiles=unit_tiles)
    h = H.to_host()
    want = reference_layout(dst, src, vals, nr, nc, min_nnz, unit_tiles or 32)
    print(f"hybrid layout nr={nr} nc={nc} nnz={nnz}: {h['num_tiles']} tiles, {h['tile_nnz']} tile entries", flush=True)
    assert h["hub_cols"] == want["hub_cols"] and h["unit_tiles"] == (unit_tiles or 32)
    for k in ("rowOrder", "hubColOrder", "rowBlockOffset", "tileCol", "units"):
        assert np.array_equal(h[k], want[k]), k
    assert np.array_equal(h["tileVals"], want["tileVals"])
    assert h["tile_nnz"] == int((~want["rest"]).sum())
    # the remainder: the oracle's BCSR of exactly the entries outside dense tiles
    rest = want["rest"]
    rd, rs = dst[rest].astype(np.int64), src[rest]
    order = np.lexsort((rs, rd))
    rowptr = np.zeros(nr + 1, np.int64)
    np.cumsum(np.bincount(rd, minlength=nr), out=rowptr[1:])
    ob = oracle.bcsr_build(nr, nc, rowptr, rs[order], None if vals is None else vals[rest][order])
    got = h["rest"]
    B = ob["num_TCBlocks"]
    assert got["num_TCBlocks"] == B and got["nnz"] == int(rest.sum())
    assert np.array_equal(got["rowWindowOffset"], ob["rowWindowOffset"])
    assert np.array_equal(got["tcOffset"], ob["tcOffset"])
    assert np.array_equal(got["sparseA2B"], ob["sparseA2B"][: 8 * B])
    assert np.array_equal(got["tcLocalBit"], ob["tcLocalBit"][:B])
    if values and got["nnz"]:
        assert np.array_equal(got["data"], ob["data"][: got["nnz"]])


CASES = [
    # nr, nc, nnz, hubs, min_nnz, unit_tiles, phases, values, F
    (500, 700, 30000, True, 32, 0, 1, True, 602),
    (500, 700, 30000, True, 32, 1, 4, True, 602),
    (500, 700, 30000, True, 8, 3, 1, False, 90),
    (1000, 900, 60000, True, 24, 0, 4, True, 256),
    (1000, 900, 60000, True, 24, 2, 1, True, 257),
    (129, 33, 2000, False, 1, 3, 1, True, 64),
    (300, 300, 5000, True, 256, 0, 1, True, 100),
    (64, 64, 4096, False, 64, 0, 1, True, 1),
    (64, 64, 4096, False, 64, 1, 1, False, 3),
    (777, 1500, 40000, True, 16, 5, 2, True, 700),
    (400, 2000, 60000, True, 4, 64, 1, True, 130),   # 64-tile units, long shared row blocks
    (60, 60, 0, False, 32, 0, 1, True, 64),
]


@pytest.mark.parametrize("nr, nc, nnz, hubs, min_nnz, unit_tiles, phases, values, F", CASES)
def test_hybrid_spmm_vs_oracle(gpu, oracle, nr, nc, nnz, hubs, min_nnz, unit_tiles, phases, values, F):
    from tcc_amd import swtcf

    print(f"hybrid nr={nr} nc={nc} nnz={nnz} min_nnz={min_nnz} unit_tiles={unit_tiles} phases={phases} "
          f"values={values} F={F}", flush=True)
    dst, src = random_coo(nr, nc, nnz, 5 * nr + nc + F, hubs)
    rng = np.random.default_rng(F + nnz + min_nnz)
    vals = rng.uniform(-1, 1, dst.size).astype(np.float32) if values else None
    X = rng.standard_normal((nc, F)).astype(np.float32)
    H = swtcf.coo_to_hybrid(dev_u32(dst), dev_u32(src), None if vals is None else torch.from_numpy(vals).cuda(), nr, nc,
                            min_tile_nnz=min_nnz, unit_tiles=unit_tiles, phases=phases)
    Xd = torch.from_numpy(X).cuda()
    Y = swtcf.hybrid_spmm(H, Xd)
    want = oracle_product(oracle, dst, src, vals, nr, X)
    got = Y.cpu().numpy()
    assert got.shape[0] >= nr
    e = rel_l2(got[:nr], want)
    assert e <= REL, f"rel-L2 {e}"
    assert not np.any(got[nr:])
    Y0 = rng.standard_normal(got.shape).astype(np.float32)
    Yd = torch.from_numpy(Y0).cuda()
    swtcf.hybrid_spmm(H, Xd, Yd, accumulate=True)
    e = rel_l2(Yd.cpu().numpy()[:nr], want + Y0[:nr])
    assert e <= REL, f"accumulate rel-L2 {e}"
    # a second product into the same Y (tiles add into the remainder's fill)
    swtcf.hybrid_spmm(H, Xd, Y)
    assert rel_l2(Y.cpu().numpy()[:nr], want) <= REL


def test_hybrid_errors(gpu):
    from tcc_amd import _lib, swtcf

    with pytest.raises(_lib.TccError, match="duplicate"):
        swtcf.coo_to_hybrid(dev_u32(np.array([0, 1, 1], np.uint32)), dev_u32(np.array([2, 3, 3], np.uint32)), None, 4, 4)
    with pytest.raises(_lib.TccError, match="out of range"):
        swtcf.coo_to_hybrid(dev_u32(np.array([0, 9], np.uint32)), dev_u32(np.array([0, 1], np.uint32)), None, 4, 4)
    with pytest.raises(_lib.TccError, match="out of range"):
        swtcf.coo_to_hybrid(dev_u32(np.array([0, 1], np.uint32)), dev_u32(np.array([0, 4], np.uint32)), None, 4, 4)
    with pytest.raises(_lib.TccError, match="unitTiles above 64"):
        swtcf.coo_to_hybrid(dev_u32(np.array([0], np.uint32)), dev_u32(np.array([1], np.uint32)), None, 4, 4,
                            unit_tiles=65)
    H = swtcf.coo_to_hybrid(dev_u32(np.array([0], np.uint32)), dev_u32(np.array([1], np.uint32)), None, 4, 4)
    X = torch.ones(4, 8, device="cuda")
    small = torch.empty(8, dtype=torch.uint8, device="cuda")
    with pytest.raises(_lib.TccError, match="workspace"):
        swtcf.hybrid_spmm(H, X, workspace=small)
