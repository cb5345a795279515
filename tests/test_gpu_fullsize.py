"""Products and conversions at BASELINE.json's full sizes.

Three checks, each able to see a misrouted row:

- Weighted checksum of checksums: for Y = A X and seeded random fp64 row
  weights r, r^T Y = (r^T A) X, i.e. per feature f
      sum_i r_i Y[i, f] = sum_j c_j X[j, f],   c_j = sum_i r_i a_ij,
  with the forward products' TF32 rounding applied to a_ij and X on the
  right.  The left side is formed on the device in fp64, the right side in
  numpy fp64 from the COO.  A partial sum landing in the wrong output row
  changes the left side by (r_i - r_k) times that sum, so the check fails on
  a swap of two output rows (planted in a copy of the result below), not
  only on missing data.  For the transposed product (plain fp32)
  s^T (A^T dY) = (A s)^T dY.
- Rows against the oracle: the fp64 CSR oracle on TF32-rounded inputs over
  a seeded sample of output rows holding at least 1M nonzeros (the hub row
  included), element by element at rel-L2 <= 1e-5 (north_star bound 1e-3).
- Every config-3 format the bench or the API offers (BCSR, 4-phase BCSR,
  valued hub tiles + remainder, binary hub tiles with the sym-norm values as
  row and column scales + remainder).
- The converter: the 114M-edge SWTCF of config 3 against the C oracle's
  canonical form, every array bit for bit.

Config 5's training step runs once at full size against a float64
evaluation of the same formulas (scipy sparse products, fp64 GEMMs).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

# Weighted checksums: measured 3e-8 to 2e-7 for the forward products, 1.4e-6
# for the F = 2 transposed product (2 sums over hub columns of ~1e5 fp32
# terms each); a swap of two output rows moves them by 6e-3 to 3e-2.
TOL = 1e-5
ROW_TOL = 1e-5  # oracle rows: measured ~1e-7 (north_star bound 1e-3)
SAMPLE_NNZ = 1_000_000


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def graph(cfg_id):
    from tcc_amd.graphs import CONFIGS, make_features, make_graph

    cfg = CONFIGS[cfg_id]
    n, F = cfg["n"], cfg["F"]
    rows, cols, vals = make_graph(cfg_id, device="cuda")
    r32 = rows.to(torch.int32).contiguous()
    c32 = cols.to(torch.int32).contiguous()
    X = make_features(n, F, cfg["seed"], device="cuda")
    return n, F, r32, c32, vals, X


def weights(n, seed):
    return np.random.default_rng(seed).standard_normal(n)


def weighted_want(oracle, rows, cols, vals, n_in, r, Xin, tf32):
    """(r^T A) X in fp64 from the COO (rows = output index of each entry)."""
    a = np.ones(rows.size, np.float64) if vals is None else vals.astype(np.float64)
    if tf32 and vals is not None:
        a = oracle.tf32(vals.astype(np.float32)).astype(np.float64)
    c = np.bincount(cols, weights=r[rows] * a, minlength=n_in)
    Xt = oracle.tf32(Xin) if tf32 else Xin
    return c @ Xt.astype(np.float64)


def weighted_got(Y, r_dev, n):
    return torch.mv(Y[:n].double().t(), r_dev).cpu().numpy()


def check_weighted(oracle, Y, n, rows, cols, vals, n_in, Xin, seed, tf32=True, what=""):
    r = weights(n, seed)
    r_dev = torch.from_numpy(r).cuda()
    want = weighted_want(oracle, rows, cols, vals, n_in, r, Xin, tf32)
    e = rel_l2(weighted_got(Y, r_dev, n), want)
    print(f"{what}: weighted checksum rel-L2 {e:.2e}", flush=True)
    assert e <= TOL, what
    return r_dev, want


def check_swap_fails(Y, n, r_dev, want, i, k, what=""):
    """A copy of Y with output rows i and k swapped fails the check (the
    planted mistake shows what the check can see)."""
    Z = Y[:n].clone()
    Z[[i, k]] = Z[[k, i]]
    e = rel_l2(weighted_got(Z, r_dev, n), want)
    print(f"{what}: rows {i} and {k} swapped: rel-L2 {e:.2e}", flush=True)
    assert e > 100 * TOL, what


def sample_rows(rows_np, n, seed, min_nnz=SAMPLE_NNZ):
    """Seeded sample of output rows holding at least min_nnz nonzeros (the
    highest-degree row first)."""
    deg = np.bincount(rows_np, minlength=n)
    rng = np.random.default_rng(seed)
    order = rng.permutation(n)
    top = int(np.argmax(deg))
    order = np.concatenate([[top], order[order != top]])
    k = int(np.searchsorted(np.cumsum(deg[order]), min_nnz)) + 1
    return np.sort(order[:k])


def check_rows(oracle, Y, rows_np, cols_np, vals_np, n, Xin, seed, what="", tf32=True):
    """Output rows of a seeded >= 1M-nnz sample against the CSR oracle
    (TF32-rounded operands for the forward products, plain fp32 for A^T)."""
    sel = sample_rows(rows_np, n, seed)
    keep = np.isin(rows_np, sel)
    r, c = rows_np[keep], cols_np[keep]
    v = None if vals_np is None else vals_np[keep]
    pos = np.searchsorted(sel, r)
    order = np.lexsort((c, pos))
    rowptr = np.zeros(sel.size + 1, np.int64)
    np.cumsum(np.bincount(pos, minlength=sel.size), out=rowptr[1:])
    want = oracle.csr_spmm(rowptr, c[order].astype(np.uint32), None if v is None else v[order], Xin, use_tf32=tf32)
    got = Y[torch.from_numpy(sel).cuda()].cpu().numpy()
    e = rel_l2(got, want)
    print(f"{what}: {sel.size} rows, {int(keep.sum())} nnz against the oracle: rel-L2 {e:.2e}", flush=True)
    assert int(keep.sum()) >= SAMPLE_NNZ
    assert e <= ROW_TOL, what


def test_fullsize_config2(gpu, oracle):
    from tcc_amd import swtcf

    n, F, r32, c32, vals, X = graph(2)
    print(f"config 2: n={n} nnz={r32.numel()} F={F}", flush=True)
    rows, cols, v = r32.cpu().numpy(), c32.cpu().numpy(), vals.cpu().numpy()
    Xh = X.cpu().numpy()
    A = swtcf.coo_to_bcsr(r32, c32, vals, n, n)
    Y = swtcf.bcsr_spmm(A, X)
    r_dev, want = check_weighted(oracle, Y, n, rows, cols, v, n, Xh, 21, what="config 2 BCSR gather")
    assert torch.count_nonzero(Y[n:]).item() == 0
    hub = int(np.argmax(np.bincount(rows, minlength=n)))
    check_swap_fails(Y, n, r_dev, want, hub, (hub + 1) % n, what="config 2")
    check_rows(oracle, Y, rows, cols, v, n, Xh, 22, what="config 2 BCSR gather")

    B = swtcf.coo_to_bcsc(r32, c32, vals, n, n)
    dY = torch.randn(n, F, device="cuda")
    dX = swtcf.bcsc_transpose_spmm(B, dY)
    # s^T (A^T dY) = (A s)^T dY: the transposed product's output index is the column
    check_weighted(oracle, dX, n, cols, rows, v, n, dY.cpu().numpy(), 23, tf32=False,
                   what="config 2 transposed gather")
    check_rows(oracle, dX, cols, rows, v, n, dY.cpu().numpy(), 24, what="config 2 transposed gather", tf32=False)


def test_fullsize_config3_bcsr(gpu, oracle):
    """The packed gather over the ordinary and the 4-phase BCSR (the bench's
    path), and the fp32 gather."""
    from tcc_amd import swtcf

    n, F, r32, c32, vals, X = graph(3)
    print(f"config 3: n={n} nnz={r32.numel()} F={F}", flush=True)
    rows, cols, v = r32.cpu().numpy(), c32.cpu().numpy(), vals.cpu().numpy()
    Xh = X.cpu().numpy()
    hub = int(np.argmax(np.bincount(rows, minlength=n)))
    P = swtcf.tf32_pack(X)
    A4 = swtcf.coo_to_bcsr(r32, c32, vals, n, n, phases=4)
    Y4 = swtcf.bcsr_spmm_packed(A4, P, F)
    r_dev, want = check_weighted(oracle, Y4, n, rows, cols, v, n, Xh, 31, what="config 3 packed, 4 phases")
    check_swap_fails(Y4, n, r_dev, want, hub, (hub + 7) % n, what="config 3")
    check_rows(oracle, Y4, rows, cols, v, n, Xh, 32, what="config 3 packed, 4 phases")
    A4.release()
    del Y4
    A1 = swtcf.coo_to_bcsr(r32, c32, vals, n, n)
    Y1 = swtcf.bcsr_spmm_packed(A1, P, F)
    check_weighted(oracle, Y1, n, rows, cols, v, n, Xh, 31, what="config 3 packed, ordinary")
    del Y1, P
    Yf = swtcf.bcsr_spmm(A1, X)
    check_weighted(oracle, Yf, n, rows, cols, v, n, Xh, 31, what="config 3 fp32 gather")


@pytest.mark.parametrize("min_nnz, G, split", [(16, 8, True), (32, 4, False)])
def test_fullsize_config3_hybrid(gpu, oracle, min_nnz, G, split):
    """The bench's path at config 3: dense hub tiles (>= 16 nnz, groups of 8
    row blocks, TF32 split into bf16 halves) on MFMA plus the packed gather of
    the remainder over its 4-phase BCSR; and the fp32-MFMA tiles (>= 32 nnz,
    groups of 4).  Y = AX and Y += AX."""
    from tcc_amd import swtcf

    n, F, r32, c32, vals, X = graph(3)
    rows, cols, v = r32.cpu().numpy(), c32.cpu().numpy(), vals.cpu().numpy()
    Xh = X.cpu().numpy()
    H = swtcf.coo_to_hybrid(r32, c32, vals, n, n, min_tile_nnz=min_nnz, group_blocks=G, phases=4,
                            tile_format=swtcf.TILES_BF16X2 if split else swtcf.TILES_FP32)
    t = H.view.tiles
    print(f"config 3 hybrid (min {min_nnz}, G {G}, split {split}): {t.num_tiles} tiles in {t.num_steps} steps, "
          f"{t.nnz} tile entries, {H.rest.view.nnz} in the remainder", flush=True)
    assert t.nnz + H.rest.view.nnz == r32.numel() and t.nnz > r32.numel() // 3
    Y = swtcf.hybrid_spmm(H, X)
    r_dev, want = check_weighted(oracle, Y, n, rows, cols, v, n, Xh, 35, what="config 3 hybrid")
    hub = int(np.argmax(np.bincount(rows, minlength=n)))
    check_swap_fails(Y, n, r_dev, want, hub, (hub + 5) % n, what="config 3 hybrid")
    check_rows(oracle, Y, rows, cols, v, n, Xh, 36, what="config 3 hybrid")
    # Y += AX over a copy of AX: 2 AX
    Y2 = Y.clone()
    swtcf.hybrid_spmm(H, X, Y2, accumulate=True)
    check_weighted(oracle, Y2 * 0.5, n, rows, cols, v, n, Xh, 35, what="config 3 hybrid, accumulate")


def test_fullsize_config3_binary_hybrid(gpu, oracle):
    """The bench's path at config 3: binary hub tiles (steps of >= 40
    entries, groups of 16 row blocks) with the sym-normalised values as row
    and column scales, plus the packed gather of the remainder's pattern
    over its 2-phase BCSR.  The reference numerics of this form are
    r_i sum_j P_ij TF32(fp32(c_j X_j)): the weighted checksum and the oracle
    rows are taken against them (rel-L2 <= 1e-5), and the oracle rows also
    against the TF32 CSR oracle over the values (north_star bound 1e-3).
    Y = AX and Y += AX."""
    from tcc_amd import swtcf
    from tcc_amd.graphs import sym_norm_scales

    n, F, r32, c32, vals, X = graph(3)
    rows_t, cols_t = r32.long(), c32.long()
    rs, cs = sym_norm_scales(rows_t, cols_t, n)
    rows, cols, v = r32.cpu().numpy(), c32.cpu().numpy(), vals.cpu().numpy()
    r_np, c_np = rs.cpu().numpy(), cs.cpu().numpy()
    H = swtcf.coo_to_hybrid_scaled(r32, c32, n, n, rs, cs, min_step_nnz=40, group_blocks=16, phases=2)
    t = H.view.tiles
    print(f"config 3 binary hybrid: {t.num_steps} steps, {t.nnz} tile entries, {H.rest.view.nnz} in the remainder, "
          f"{t.num_units} units ({t.num_partial_units} with partial sums)", flush=True)
    assert t.nnz + H.rest.view.nnz == r32.numel() and t.nnz > r32.numel() // 2
    Y = swtcf.hybrid_spmm(H, X)
    Xh = X.cpu().numpy()
    Xs = oracle.tf32((Xh * c_np[:, None]).astype(np.float32))  # TF32(fp32(c_j X_j))
    w = weights(n, 37)
    w_dev = torch.from_numpy(w).cuda()
    want = np.bincount(cols, weights=w[rows] * r_np[rows].astype(np.float64), minlength=n) @ Xs.astype(np.float64)
    e = rel_l2(weighted_got(Y, w_dev, n), want)
    print(f"config 3 binary hybrid: weighted checksum rel-L2 {e:.2e}", flush=True)
    assert e <= TOL
    hub = int(np.argmax(np.bincount(rows, minlength=n)))
    check_swap_fails(Y, n, w_dev, want, hub, (hub + 5) % n, what="config 3 binary hybrid")
    # oracle rows: the pattern over TF32(c X), times r
    sel = sample_rows(rows, n, 38)
    keep = np.isin(rows, sel)
    rr, cc, vv = rows[keep], cols[keep], v[keep]
    pos = np.searchsorted(sel, rr)
    order = np.lexsort((cc, pos))
    rowptr = np.zeros(sel.size + 1, np.int64)
    np.cumsum(np.bincount(pos, minlength=sel.size), out=rowptr[1:])
    ref = oracle.csr_spmm(rowptr, cc[order].astype(np.uint32), None, Xs, use_tf32=True) * \
        r_np[sel, None].astype(np.float64)
    got = Y[torch.from_numpy(sel).cuda()].cpu().numpy()
    e = rel_l2(got, ref)
    ref_v = oracle.csr_spmm(rowptr, cc[order].astype(np.uint32), vv[order], Xh, use_tf32=True)
    e_v = rel_l2(got, ref_v)
    print(f"config 3 binary hybrid: {sel.size} rows, {int(keep.sum())} nnz: rel-L2 {e:.2e} against r TF32(c X), "
          f"{e_v:.2e} against the TF32 CSR oracle over the values", flush=True)
    assert int(keep.sum()) >= SAMPLE_NNZ
    assert e <= ROW_TOL
    assert e_v <= 1e-3
    Y2 = Y.clone()
    swtcf.hybrid_spmm(H, X, Y2, accumulate=True)
    e = rel_l2(weighted_got(Y2 * 0.5, w_dev, n), want)
    print(f"config 3 binary hybrid, accumulate: weighted checksum rel-L2 {e:.2e}", flush=True)
    assert e <= TOL


def _extension():
    import os
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    sys.path.insert(0, os.path.join(root, "tcc_amd"))
    try:
        import spmm_cnic
    finally:
        sys.path.pop(0)
    return spmm_cnic


def _ext_args(d, kind):
    """The 9 (or 10 with data) tensor/int arguments of one matrix in the
    reference's extension call (train/tcgnn_conv_release.py:116-130)."""
    def dev(a):
        a = np.ascontiguousarray(a)
        return torch.from_numpy(a.view(np.int32) if a.dtype == np.uint32 else
                                (a.view(np.int64) if a.dtype == np.uint64 else a)).cuda()

    w = "rowWindowOffset" if kind == "bcsr" else "colWindowOffset"
    i = "sparseA2B" if kind == "bcsr" else "sparseA2C"
    nw = d["num_rowWindows"] if kind == "bcsr" else d["num_colWindows"]
    data = d["data"] if d["data"] is not None else np.zeros(1, np.float32)
    return [d["num_rows"], d["num_cols"], d["nnz"], d["num_TCBlocks"], nw, dev(d[w]), dev(d["tcOffset"]), dev(d[i]),
            dev(d["tcLocalBit"]), dev(data)]


def test_fullsize_config3_extension(gpu, oracle):
    """spmm_cnic.forward_tensorcore, called as the reference's training
    script calls it, on config 3's BCSR (the whole graph; an empty BCSC;
    values not read, as the reference's kernels read none): the default path
    (x packed to exact TF32 rows, the packed gather) and a per-graph plan
    (set_graph_plans: binary tiles + gather); each against >= 1M-nnz oracle
    rows of the pattern product and the weighted checksum."""
    from tcc_amd import swtcf

    m = _extension()
    n, F, r32, c32, vals, X = graph(3)
    rows, cols = r32.cpu().numpy(), c32.cpu().numpy()
    Xh = X.cpu().numpy()
    A = swtcf.coo_to_bcsr(r32, c32, None, n, n)
    B = swtcf.coo_to_bcsc(r32[:0], c32[:0], None, n, n)
    args = _ext_args(A.to_host(), "bcsr") + _ext_args(B.to_host(), "bcsc")
    A.release()
    x = X.flatten()
    hub = int(np.argmax(np.bincount(rows, minlength=n)))
    try:
        for plans in (0, 1):
            m.set_graph_plans(plans)
            out = m.forward_tensorcore(*args, F, x)
            Y = out.reshape(n, F)
            what = f"config 3 forward_tensorcore, {'a per-graph plan' if plans else 'packed x'}"
            r_dev, want = check_weighted(oracle, Y, n, rows, cols, None, n, Xh, 39, what=what)
            check_swap_fails(Y, n, r_dev, want, hub, (hub + 9) % n, what=what)
            check_rows(oracle, Y, rows, cols, None, n, Xh, 40, what=what)
            if plans:
                assert m.graph_plans() == 1
            m.freeMatC()
    finally:
        m.set_graph_plans(-1)
        m.freeMatC()


def test_fullsize_config3_swtcf_bit_exact(gpu, oracle):
    """convertCOOToSWTCF of the config-3 graph (114M edges, S = 16) against
    the C oracle's canonical form, every array bit for bit, for the COO in
    the generator's (dst, src) order (the sort's super-window digits alone
    order it) and for the same COO under a seeded permutation (every digit
    runs: the per-super-window low passes of a COO out of order); the
    canonical form does not depend on the input order.  Then the SWTCF SpMM
    (F = 128) through the weighted checksum."""
    from tcc_amd import swtcf
    from tcc_amd.graphs import CONFIGS, make_graph

    n = CONFIGS[3]["n"]
    rows, cols, _ = make_graph(3, device="cuda")
    r32 = rows.to(torch.int32).contiguous()
    c32 = cols.to(torch.int32).contiguous()
    del rows, cols
    nnz = r32.numel()
    print(f"config 3 SWTCF: n={n} nnz={nnz}", flush=True)
    m = swtcf.DeviceSWTCFMatrix(n, n, nnz, 16)
    ws = swtcf.SWTCFConvertWorkspace(nnz, n, 16)
    swtcf.convertCOOToSWTCF(r32, c32, nnz, m, ws)
    assert ws.device_error() == 0
    got = m.to_host()
    dst = r32.cpu().numpy().view(np.uint32)
    src = c32.cpu().numpy().view(np.uint32)
    print("oracle conversion (host)...", flush=True)
    ref = oracle.swtcf_convert(dst, src, n, n, 16)
    assert ref["err"] == 0
    want = oracle.swtcf_valid_extents(ref)
    del ref
    for k, vv in want.items():
        assert np.array_equal(got[k], vv), f"SWTCF array {k} differs from the oracle"
    print(f"bit-exact: {got['numTiles']} tiles, {got['numRows']} super-window rows", flush=True)
    del got
    perm = torch.randperm(nnz, device="cuda", generator=torch.Generator(device="cuda").manual_seed(77))
    ms = swtcf.DeviceSWTCFMatrix(n, n, nnz, 16)
    swtcf.convertCOOToSWTCF(r32[perm].contiguous(), c32[perm].contiguous(), nnz, ms, ws)
    del perm
    assert ws.device_error() == 0
    got = ms.to_host()
    for k, vv in want.items():
        assert np.array_equal(got[k], vv), f"SWTCF array {k} of the shuffled COO differs from the oracle"
    print("shuffled COO: bit-exact", flush=True)
    ms.free()
    del want, got

    F = 128
    Xh = oracle.tf32(np.random.default_rng(35).standard_normal((n, F)).astype(np.float32))
    Ys = torch.zeros(n, F, device="cuda")
    swtcf.swtcf_spmm(m, torch.from_numpy(Xh).cuda(), Ys, 12)
    check_weighted(oracle, Ys, n, dst, src, None, n, Xh, 36, what="config 3 SWTCF SpMM")


def test_fullsize_config4_mixed_and_narrow(gpu, oracle):
    """The GCN graph (2.45M nodes, 61.9M edges, every a_ij = 1): the
    first-layer product over the hot/cold feature table (fp32 and packed
    host rows), the second layer's F = 2 product and its transpose."""
    from tcc_amd import gcn, swtcf
    from tcc_amd.graphs import CONFIGS, make_features, make_graph

    cfg = CONFIGS[4]
    n, F = cfg["n"], cfg["F"]
    rows, cols, _ = make_graph(4, device="cuda")
    print(f"config 4: n={n} nnz={rows.numel()} F={F}", flush=True)
    X = make_features(n, F, cfg["seed"], device="cuda")
    Xh = X.cpu().numpy()
    rows_np, cols_np = rows.cpu().numpy(), cols.cpu().numpy()
    table = gcn.FeatureTable(X, cols)
    g1, g2 = gcn.build_gcn_graphs(rows, cols, n, table.hot)
    hub = int(np.argmax(np.bincount(rows_np, minlength=n)))

    Y = g1.aggregate(F, source=table.source)
    r_dev, want = check_weighted(oracle, Y, n, rows_np, cols_np, None, n, Xh, 41, what="config 4 mixed, fp32 rows")
    check_swap_fails(Y, n, r_dev, want, hub, (hub + 5) % n, what="config 4 mixed")
    check_rows(oracle, Y, rows_np, cols_np, None, n, Xh, 42, what="config 4 mixed, fp32 rows")
    assert table.error() == 0
    del Y
    ptable = gcn.FeatureTable(X, cols, packed=True)
    Yp = g1.aggregate(F, source=ptable.source)
    check_weighted(oracle, Yp, n, rows_np, cols_np, None, n, Xh, 41, what="config 4 mixed, packed rows")
    check_rows(oracle, Yp, rows_np, cols_np, None, n, Xh, 43, what="config 4 mixed, packed rows")
    assert ptable.error() == 0
    del Yp
    ptable.free()

    XW = torch.randn(n, 2, device="cuda")
    Y2 = g2.aggregate(2, x=XW)
    check_weighted(oracle, Y2, n, rows_np, cols_np, None, n, XW.cpu().numpy(), 44, what="config 4 narrow F=2")
    dY = torch.randn(n, 2, device="cuda")
    dX = swtcf.bcsc_transpose_spmm(g2.bwd, dY)
    check_weighted(oracle, dX, n, cols_np, rows_np, None, n, dY.cpu().numpy(), 45, tf32=False,
                   what="config 4 narrow transpose F=2")
    check_rows(oracle, dX, cols_np, rows_np, None, n, dY.cpu().numpy(), 46, what="config 4 narrow transpose F=2",
               tf32=False)
    check_rows(oracle, Y2, rows_np, cols_np, None, n, XW.cpu().numpy(), 47, what="config 4 narrow F=2")
    table.free()


def test_fullsize_config5_training_step(gpu):
    """One full-graph training step of the 2-layer GCN (100 -> 256 -> 2) on
    the 2.45M-node graph, fused path (TwoLayerFunction), against a float64
    evaluation of the same formulas: scipy fp64 sparse products with the
    kernels' rounding (TF32 into the forward SpMMs, fp32 into A^T), fp64
    GEMMs.  rel-L2 <= 1e-4 as the small-graph test."""
    import scipy.sparse as sp

    from tcc_amd import gcn
    from tcc_amd.graphs import CONFIGS, make_features, make_graph

    cfg = CONFIGS[5]
    n, F, Hd, C = cfg["n"], cfg["F"], 256, 2
    rows, cols, _ = make_graph(5, device="cuda")
    print(f"config 5: n={n} nnz={rows.numel()} F={F} hidden={Hd} classes={C}", flush=True)
    X = make_features(n, F, cfg["seed"], device="cuda")
    table = gcn.FeatureTable(X, cols)
    g1, g2 = gcn.build_gcn_graphs(rows, cols, n, table.hot)
    torch.manual_seed(cfg["seed"])
    model = gcn.GCN(F, Hd, C, dropout=0.0).cuda()
    assert model.fused
    labels = gcn.synthetic_labels(n, C, cfg["seed"])
    W1 = model.conv1.weights.detach().double()
    W2 = model.conv_final.weights.detach().double()
    pred = model(g1, g2, table.source)
    loss = gcn.cross_entropy(pred, labels)
    loss.backward()
    torch.cuda.synchronize()
    assert table.error() == 0

    def tf32(t):
        b = t.float().contiguous().view(torch.int32)
        fin = (b & 0x7F800000) != 0x7F800000
        r = torch.where(fin, (b + 0x1000) & -0x2000, b)
        return r.view(torch.float32).double()

    A = sp.csr_matrix((np.ones(rows.numel()), (rows.cpu().numpy(), cols.cpu().numpy())), shape=(n, n))
    At = A.T.tocsr()
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    AX1 = dev(A @ tf32(X).cpu().numpy())
    H1 = AX1 @ W1
    R = torch.clamp_min(H1, 0.0)
    out = dev(A @ tf32(R @ W2).cpu().numpy())
    logp = torch.log_softmax(out, dim=1)
    ref_loss = -logp[torch.arange(n, device="cuda"), labels].mean()
    dout = torch.softmax(out, dim=1)
    dout[torch.arange(n, device="cuda"), labels] -= 1.0
    dout /= n
    G2 = dev(At @ dout.float().double().cpu().numpy())
    dW2 = R.t() @ G2
    dH1 = (G2 @ W2.t()) * (H1 > 0)
    dW1 = AX1.t() @ dH1
    e_out = rel_l2(pred.detach().double().cpu().numpy(), out.cpu().numpy())
    e_dw1 = rel_l2(model.conv1.weights.grad.double().cpu().numpy(), dW1.cpu().numpy())
    e_dw2 = rel_l2(model.conv_final.weights.grad.double().cpu().numpy(), dW2.cpu().numpy())
    print(f"config 5 step: out {e_out:.2e}, loss {loss.item():.6f} vs {ref_loss.item():.6f}, dW1 {e_dw1:.2e}, "
          f"dW2 {e_dw2:.2e}", flush=True)
    assert e_out < 1e-4
    assert abs(loss.item() - ref_loss.item()) < 1e-4 * abs(ref_loss.item())
    assert e_dw1 < 1e-4
    assert e_dw2 < 1e-4
    table.free()
