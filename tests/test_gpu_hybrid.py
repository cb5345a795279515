"""Dense hub tiles + sparse remainder (tcc_coo_to_hybrid, tcc_hybrid_spmm).

Checked through the C-ABI:
- the arrays, exactly, against an independent numpy construction of the
  layout include/tcc_spmm_cnic.h states: rows and columns ranked by degree
  (descending, then index); 16x16 tiles of the reordered matrix with at
  least min_tile_nnz entries; steps = the (group of G row blocks, column
  block) pairs holding one, sorted; values TF32-rounded at A(row l%16,
  column 4s + l/16) -> tileVals[step][row block % G][l][s], zeros in the
  other slots; units of unit_steps steps and their launch order (by the
  column block of their first step, stable); the other entries' BCSR equal
  to the oracle's BCSR of exactly those entries;
- the products against the fp64 CSR oracle on TF32-rounded inputs (rel-L2
  <= 1e-5) for both tile formats (fp32 A operand; TF32 split into two bf16,
  four exact bf16 products), in a workspace of NaN bytes, Y = AX and Y += AX,
  the units launched in their stored order or (NULL order) in index order,
  over thresholds from 1 (every tile dense) to
  256 (no tile dense), groups of 1, 2, 4 and 8 row blocks (row counts that
  leave the last group partly empty), groups shared by many units (their
  partial sums reduced in a second pass), unit sizes 1 to 256, phased
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


DEFAULT_UNIT_STEPS = 128  # the builder's unitSteps = 0


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


def bf16_split(x):
    """hi = top 16 bits of the TF32 value, lo = top 16 bits of the exact remainder (0 for inf/NaN)."""
    b = np.asarray(x, np.float32).view(np.uint32)
    hi = (b >> 16).astype(np.uint16)
    rest = (np.asarray(x, np.float32) - (b & 0xFFFF0000).view(np.float32)).view(np.uint32)
    lo = np.where((b & 0x7F800000) == 0x7F800000, 0, rest >> 16).astype(np.uint16)
    return hi, lo


def reference_layout(dst, src, vals, nr, nc, min_nnz, G, unit_steps, split=False):
    dst = dst.astype(np.int64)
    src = src.astype(np.int64)
    rorder = np.lexsort((np.arange(nr), -np.bincount(dst, minlength=nr)))
    corder = np.lexsort((np.arange(nc), -np.bincount(src, minlength=nc)))
    rrank = np.empty(nr, np.int64)
    rrank[rorder] = np.arange(nr)
    crank = np.empty(nc, np.int64)
    crank[corder] = np.arange(nc)
    RB, CB = (nr + 15) // 16, (nc + 15) // 16
    NG = (RB + G - 1) // G
    row_order = np.full(16 * G * NG, 0xFFFFFFFF, np.uint32)
    row_order[:nr] = rorder
    rr, cr = rrank[dst], crank[src]
    rb, cb = rr // 16, cr // 16
    tile = rb * CB + cb
    keys, counts = np.unique(tile, return_counts=True)
    dense_keys = keys[counts >= min_nnz]
    in_dense = np.isin(tile, dense_keys)
    step_keys = np.unique((dense_keys // CB) // G * CB + dense_keys % CB)  # (group, column block), sorted
    S = step_keys.size
    sid = np.searchsorted(step_keys, (rb[in_dense] // G) * CB + cb[in_dense])
    vals_all = np.ones(dst.size, np.float32) if vals is None else vals
    i, j = rr[in_dense] % 16, cr[in_dense] % 16
    if split:  # [step][row block][hi, lo][row][column], bf16 bits
        tv = np.zeros((S, G, 2, 16, 16), np.uint16)
        hi, lo = bf16_split(tf32(vals_all[in_dense]))
        tv[sid, rb[in_dense] % G, 0, i, j] = hi
        tv[sid, rb[in_dense] % G, 1, i, j] = lo
    else:  # the fp32 MFMA's A operand: [step][row block][lane][k-step]
        tv = np.zeros((S, G, 64, 4), np.float32)
        tv[sid, rb[in_dense] % G, i + 16 * (j % 4), j // 4] = tf32(vals_all[in_dense])
    sg, sc = step_keys // CB, step_keys % CB
    gso = np.searchsorted(sg, np.arange(NG + 1)).astype(np.uint32)
    units = []
    for g in range(NG):
        p0, p1 = int(gso[g]), int(gso[g + 1])
        for k in range(-(-(p1 - p0) // unit_steps)):
            units.append((g, p0 + k * unit_steps, min(p0 + (k + 1) * unit_steps, p1)))
    hub_cols = min(16 * (int(sc.max()) + 1), nc) if S else 0
    units = np.array(units, np.uint32).reshape(-1, 3)
    # launch order: by the column block of each unit's first step, ties in unit order
    unit_order = np.argsort(sc[units[:, 1]] if len(units) else units[:, 1], kind="stable").astype(np.uint32)
    return dict(rowOrder=row_order, hubColOrder=corder[:hub_cols].astype(np.uint32), groupStepOffset=gso,
                stepCol=sc.astype(np.uint32), tileVals=tv, units=units, unitOrder=unit_order,
                hub_cols=hub_cols, num_tiles=int(dense_keys.size), rest=~in_dense)


def oracle_product(oracle, dst, src, vals, nr, X):
    order = np.lexsort((src, dst))
    rowptr = np.zeros(nr + 1, np.int64)
    np.cumsum(np.bincount(dst.astype(np.int64), minlength=nr), out=rowptr[1:])
    return oracle.csr_spmm(rowptr, src[order], None if vals is None else vals[order], X, use_tf32=True)


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("nr, nc, nnz, hubs, min_nnz, G, unit_steps, values", [
    (500, 700, 30000, True, 32, 4, 4, True),
    (500, 700, 30000, True, 8, 8, 0, False),
    (129, 33, 2000, False, 1, 2, 3, True),     # every occupied tile dense; a partly empty last group
    (300, 300, 5000, True, 256, 4, 0, True),   # no tile dense: all in the remainder
    (17, 1000, 3000, True, 20, 1, 1, True),
    (40, 900, 9000, True, 6, 8, 64, True),     # fewer rows than one group
    (300, 4000, 60000, True, 4, 8, 100, True),  # units past 64 steps (the second register of step columns)
    (60, 60, 0, False, 32, 0, 0, True),
])
def test_arrays_match_numpy_layout(gpu, oracle, nr, nc, nnz, hubs, min_nnz, G, unit_steps, values, split):
    from tcc_amd import swtcf

    dst, src = random_coo(nr, nc, nnz, nr * 3 + nc + nnz, hubs)
    vals = np.random.default_rng(9).uniform(-1, 1, dst.size).astype(np.float32) if values else None
    H = swtcf.coo_to_hybrid(dev_u32(dst), dev_u32(src), None if vals is None else torch.from_numpy(vals).cuda(), nr, nc,
                            min_tile_nnz=min_nnz, group_blocks=G, unit_steps=unit_steps,
                            tile_format=swtcf.TILES_BF16X2 if split else swtcf.TILES_FP32)
    h = H.to_host()
    want = reference_layout(dst, src, vals, nr, nc, min_nnz, G or 8, unit_steps or DEFAULT_UNIT_STEPS, split)
    assert h["tile_format"] == (1 if split else 0)
    print(f"hybrid layout nr={nr} nc={nc} nnz={nnz} G={G}: {h['num_steps']} steps, {h['num_tiles']} tiles, "
          f"{h['tile_nnz']} tile entries", flush=True)
    assert h["group_blocks"] == (G or 8) and h["unit_steps"] == (unit_steps or DEFAULT_UNIT_STEPS)
    assert h["hub_cols"] == want["hub_cols"] and h["num_tiles"] == want["num_tiles"]
    for k in ("rowOrder", "hubColOrder", "groupStepOffset", "stepCol", "units", "unitOrder"):
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
    # nr, nc, nnz, hubs, min_nnz, G, unit_steps, phases, values, F
    (500, 700, 30000, True, 32, 4, 0, 1, True, 602),
    (500, 700, 30000, True, 32, 4, 1, 4, True, 602),
    (500, 700, 30000, True, 8, 2, 3, 1, False, 90),
    (1000, 900, 60000, True, 24, 8, 0, 4, True, 256),
    (1000, 900, 60000, True, 24, 1, 2, 1, True, 257),
    (129, 33, 2000, False, 1, 8, 3, 1, True, 64),
    (300, 300, 5000, True, 256, 4, 0, 1, True, 100),
    (64, 64, 4096, False, 64, 4, 0, 1, True, 1),
    (64, 64, 4096, False, 64, 2, 1, 1, False, 3),
    (777, 1500, 40000, True, 16, 4, 5, 2, True, 700),
    (400, 2000, 60000, True, 4, 8, 64, 1, True, 130),   # 64-step units, long shared groups
    (400, 4000, 120000, True, 4, 8, 0, 1, True, 130),   # 128-step units (the default), long shared groups
    (400, 4000, 120000, True, 4, 4, 100, 2, True, 70),  # 100-step units
    (400, 8000, 200000, True, 4, 8, 256, 1, True, 96),  # 256-step units: all four registers of step columns
    (40, 900, 9000, True, 6, 8, 7, 1, True, 48),        # fewer rows than one group
    (60, 60, 0, False, 32, 4, 0, 1, True, 64),
]


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("nr, nc, nnz, hubs, min_nnz, G, unit_steps, phases, values, F", CASES)
def test_hybrid_spmm_vs_oracle(gpu, oracle, nr, nc, nnz, hubs, min_nnz, G, unit_steps, phases, values, F, split):
    from tcc_amd import swtcf

    print(f"hybrid nr={nr} nc={nc} nnz={nnz} min_nnz={min_nnz} G={G} unit_steps={unit_steps} phases={phases} "
          f"values={values} F={F} split={split}", flush=True)
    dst, src = random_coo(nr, nc, nnz, 5 * nr + nc + F, hubs)
    rng = np.random.default_rng(F + nnz + min_nnz)
    vals = rng.uniform(-1, 1, dst.size).astype(np.float32) if values else None
    X = rng.standard_normal((nc, F)).astype(np.float32)
    H = swtcf.coo_to_hybrid(dev_u32(dst), dev_u32(src), None if vals is None else torch.from_numpy(vals).cuda(), nr, nc,
                            min_tile_nnz=min_nnz, group_blocks=G, unit_steps=unit_steps, phases=phases,
                            tile_format=swtcf.TILES_BF16X2 if split else swtcf.TILES_FP32)
    Xd = torch.from_numpy(X).cuda()
    # a workspace of NaN bytes: no product may read what it did not write
    ws = torch.full((H.workspace_bytes(F) + 16,), 255, dtype=torch.uint8, device="cuda")
    Y = swtcf.hybrid_spmm(H, Xd, workspace=ws)
    want = oracle_product(oracle, dst, src, vals, nr, X)
    got = Y.cpu().numpy()
    assert got.shape[0] >= nr
    e = rel_l2(got[:nr], want)
    assert e <= REL, f"rel-L2 {e}"
    assert not np.any(got[nr:])
    Y0 = rng.standard_normal(got.shape).astype(np.float32)
    Yd = torch.from_numpy(Y0).cuda()
    swtcf.hybrid_spmm(H, Xd, Yd, accumulate=True, workspace=ws)
    e = rel_l2(Yd.cpu().numpy()[:nr], want + Y0[:nr])
    assert e <= REL, f"accumulate rel-L2 {e}"
    # a second product into the same Y (tiles add into the remainder's fill)
    swtcf.hybrid_spmm(H, Xd, Y, workspace=ws)
    assert rel_l2(Y.cpu().numpy()[:nr], want) <= REL
    # without a launch order (NULL: units in index order); not bit for bit,
    # since the remainder's split windows add through fp32 atomics
    order = H.view.tiles.unitOrder
    H.view.tiles.unitOrder = None
    try:
        Yn = swtcf.hybrid_spmm(H, Xd, workspace=ws)
    finally:
        H.view.tiles.unitOrder = order
    assert rel_l2(Yn.cpu().numpy()[:nr], want) <= REL


def test_hybrid_errors(gpu):
    from tcc_amd import _lib, swtcf

    with pytest.raises(_lib.TccError, match="duplicate"):
        swtcf.coo_to_hybrid(dev_u32(np.array([0, 1, 1], np.uint32)), dev_u32(np.array([2, 3, 3], np.uint32)), None, 4, 4)
    with pytest.raises(_lib.TccError, match="out of range"):
        swtcf.coo_to_hybrid(dev_u32(np.array([0, 9], np.uint32)), dev_u32(np.array([0, 1], np.uint32)), None, 4, 4)
    with pytest.raises(_lib.TccError, match="out of range"):
        swtcf.coo_to_hybrid(dev_u32(np.array([0, 1], np.uint32)), dev_u32(np.array([0, 4], np.uint32)), None, 4, 4)
    with pytest.raises(_lib.TccError, match="unitSteps above 256"):
        swtcf.coo_to_hybrid(dev_u32(np.array([0], np.uint32)), dev_u32(np.array([1], np.uint32)), None, 4, 4,
                            unit_steps=257)
    with pytest.raises(_lib.TccError, match="tileFormat"):
        swtcf.coo_to_hybrid(dev_u32(np.array([0], np.uint32)), dev_u32(np.array([1], np.uint32)), None, 4, 4,
                            tile_format=2)
    with pytest.raises(_lib.TccError, match="groupBlocks"):
        swtcf.coo_to_hybrid(dev_u32(np.array([0], np.uint32)), dev_u32(np.array([1], np.uint32)), None, 4, 4,
                            group_blocks=3)
    H = swtcf.coo_to_hybrid(dev_u32(np.array([0], np.uint32)), dev_u32(np.array([1], np.uint32)), None, 4, 4)
    X = torch.ones(4, 8, device="cuda")
    small = torch.empty(8, dtype=torch.uint8, device="cuda")
    with pytest.raises(_lib.TccError, match="workspace"):
        swtcf.hybrid_spmm(H, X, workspace=small)


def test_split_tiles_inf_in_hub_column(gpu, oracle):
    """Valued (split-TF32) tiles multiply every tile slot of a step, zeros
    included: an Inf in a hub column's feature row gives NaN to the rows
    without an entry in that column in every group with a step in its column
    block (0 * Inf in the tiles' products), Inf or NaN to those with one
    there (NaN when the value's low bf16 half is 0: al * Inf), Inf to rows
    whose entry is in the remainder, and leaves every other row finite and
    exact."""
    from tcc_amd import swtcf

    nr, nc, F, G = 400, 500, 8, 8
    dst, src = random_coo(nr, nc, 20000, 23, True)
    vals = np.random.default_rng(2).uniform(0.5, 1.5, dst.size).astype(np.float32)
    H = swtcf.coo_to_hybrid(dev_u32(dst), dev_u32(src), torch.from_numpy(vals).cuda(), nr, nc, min_tile_nnz=16,
                            group_blocks=G, tile_format=swtcf.TILES_BF16X2)
    h = H.to_host()
    c0 = int(h["hubColOrder"][0])  # rank 0: column block 0
    X = np.random.default_rng(5).standard_normal((nc, F)).astype(np.float32)
    X[c0, 0] = np.inf
    Y = swtcf.hybrid_spmm(H, torch.from_numpy(X).cuda()).cpu().numpy()[:nr]
    has = np.zeros(nr, bool)
    has[dst[src == c0].astype(np.int64)] = True
    exposed = np.zeros(nr, bool)
    gso, steps = h["groupStepOffset"], h["stepCol"]
    for g in range(h["num_groups"]):
        if np.any(steps[gso[g]:gso[g + 1]] == 0):
            rows = h["rowOrder"][16 * G * g: 16 * G * (g + 1)]
            exposed[rows[rows != 0xFFFFFFFF].astype(np.int64)] = True
    assert has.any() and (exposed & ~has).any()
    assert np.all(np.isposinf(Y[has & ~exposed, 0]))
    assert np.all(np.isposinf(Y[has & exposed, 0]) | np.isnan(Y[has & exposed, 0]))
    assert np.all(np.isnan(Y[exposed & ~has, 0]))
    assert np.all(np.isfinite(Y[~(has | exposed), 0]))
    X[c0, 0] = 0.0
    want = oracle_product(oracle, dst, src, vals, nr, X)
    keep = ~(has | exposed)
    assert rel_l2(Y[:, 1:], want[:, 1:]) <= REL
    assert rel_l2(Y[keep, 0], want[keep, 0]) <= REL
