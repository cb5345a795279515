"""Products at BASELINE.json's full sizes, through size-independent
properties (the oracle's CSR SpMM would take minutes here).

Checksum of checksums: for Y = A X, the column sums of Y satisfy
1^T Y = (1^T A) X, so per feature f
    sum_i Y[i, f] = sum_j c_j X[j, f],   c_j = sum_i a_ij,
with the forward products' TF32 rounding applied to a_ij and X on the right
(the oracle's tf32).  The left side is summed on the device in fp64; the
right side in numpy fp64 from the COO.  A missing or doubled window or unit
moves the checksum by ~1e-3 relative (config 2: one 31-edge window, 2e-3;
a single edge ~7e-5); the products agree with it to 1e-8 to 3e-8.  For the transposed product (plain fp32), 1^T (A^T dY) = (A 1)^T dY.
Config 3 also checks the 4-phase BCSR against the ordinary one, element by
element.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

TOL = 1e-6  # measured 1e-8 to 3e-8; one window of 31 edges left out moves it by 2e-3


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
    X = make_features(n, F, cfg_id, device="cuda")
    return n, F, r32, c32, vals, X


def column_sums(oracle, idx, vals, n, tf32):
    v = vals.cpu().numpy().astype(np.float32)
    if tf32:
        v = oracle.tf32(v)
    return np.bincount(idx.cpu().numpy().astype(np.int64), weights=v.astype(np.float64), minlength=n)


def device_checksum(Y, rows):
    return Y[:rows].double().sum(dim=0).cpu().numpy()


def test_fullsize_config2_checksums(gpu, oracle):
    from tcc_amd import swtcf

    n, F, r32, c32, vals, X = graph(2)
    print(f"config 2: n={n} nnz={r32.numel()} F={F}", flush=True)
    A = swtcf.coo_to_bcsr(r32, c32, vals, n, n)
    Y = swtcf.bcsr_spmm(A, X)
    c = column_sums(oracle, c32, vals, n, tf32=True)
    Xt = oracle.tf32(X.cpu().numpy()).astype(np.float64)
    want = c @ Xt
    got = device_checksum(Y, n)
    print(f"forward checksum rel-L2 {rel_l2(got, want):.2e}", flush=True)
    assert rel_l2(got, want) <= TOL, "forward"
    assert torch.count_nonzero(Y[n:]).item() == 0
    # the check's reach: the expected side without one row window's edges
    # (a mistake planted in the reference, not in the product) must fail it
    rows_np = r32.cpu().numpy()
    drop = (rows_np // 8) == 1000
    assert drop.any()
    vals_kept = torch.where(torch.from_numpy(drop).cuda(), torch.zeros_like(vals), vals)
    c_drop = column_sums(oracle, c32, vals_kept, n, tf32=True)
    miss = rel_l2(got, c_drop @ Xt)
    print(f"one window ({int(drop.sum())} edges) left out of the reference: rel-L2 {miss:.2e}", flush=True)
    assert miss > 100 * TOL

    B = swtcf.coo_to_bcsc(r32, c32, vals, n, n)
    dY = torch.randn(n, F, device="cuda")
    dX = swtcf.bcsc_transpose_spmm(B, dY)
    r = column_sums(oracle, r32, vals, n, tf32=False)  # row sums of A
    wantT = r @ dY.cpu().numpy().astype(np.float64)
    print(f"transpose checksum rel-L2 {rel_l2(device_checksum(dX, n), wantT):.2e}", flush=True)
    assert rel_l2(device_checksum(dX, n), wantT) <= TOL, "transpose"


def test_fullsize_config3_packed_phased(gpu, oracle):
    from tcc_amd import swtcf

    n, F, r32, c32, vals, X = graph(3)
    print(f"config 3: n={n} nnz={r32.numel()} F={F}", flush=True)
    c = column_sums(oracle, c32, vals, n, tf32=True)
    want = c @ oracle.tf32(X.cpu().numpy()).astype(np.float64)
    P = swtcf.tf32_pack(X)
    del X
    A4 = swtcf.coo_to_bcsr(r32, c32, vals, n, n, phases=4)
    Y4 = swtcf.bcsr_spmm_packed(A4, P, F)
    print(f"4 phases: checksum rel-L2 {rel_l2(device_checksum(Y4, n), want):.2e}", flush=True)
    assert rel_l2(device_checksum(Y4, n), want) <= TOL, "4 phases"
    A4.release()
    A1 = swtcf.coo_to_bcsr(r32, c32, vals, n, n)
    Y1 = swtcf.bcsr_spmm_packed(A1, P, F)
    assert rel_l2(device_checksum(Y1, n), want) <= TOL, "ordinary"
    d = ((Y4[:n].double() - Y1[:n].double()).norm() / Y1[:n].double().norm()).item()
    print(f"phased against ordinary: rel-L2 {d:.2e}", flush=True)
    assert d <= 1e-6, f"phased against ordinary: {d}"


def test_fullsize_config4_mixed_and_narrow(gpu, oracle):
    """The GCN graph (2.45M nodes, 61.9M edges, no values: every a_ij = 1):
    the first-layer product over the hot/cold feature table (fp32 and packed
    host rows), the second layer's F = 2 product and its transpose."""
    from tcc_amd import gcn, swtcf
    from tcc_amd.graphs import CONFIGS, make_features, make_graph

    cfg = CONFIGS[4]
    n, F = cfg["n"], cfg["F"]
    rows, cols, _ = make_graph(4, device="cuda")
    print(f"config 4: n={n} nnz={rows.numel()} F={F}", flush=True)
    X = make_features(n, F, cfg["seed"], device="cuda")
    table = gcn.FeatureTable(X, cols)
    g1, g2 = gcn.build_gcn_graphs(rows, cols, n, table.hot)
    indeg = np.bincount(cols.cpu().numpy().astype(np.int64), minlength=n).astype(np.float64)
    outdeg = np.bincount(rows.cpu().numpy().astype(np.int64), minlength=n).astype(np.float64)
    want = indeg @ oracle.tf32(X.cpu().numpy()).astype(np.float64)

    got = g1.aggregate(F, source=table.source).double().sum(dim=0).cpu().numpy()
    print(f"mixed, fp32 host rows: checksum rel-L2 {rel_l2(got, want):.2e}", flush=True)
    assert rel_l2(got, want) <= TOL, "mixed fp32"
    ptable = gcn.FeatureTable(X, cols, packed=True)
    got = g1.aggregate(F, source=ptable.source).double().sum(dim=0).cpu().numpy()
    print(f"mixed, packed host rows: checksum rel-L2 {rel_l2(got, want):.2e}", flush=True)
    assert rel_l2(got, want) <= TOL, "mixed packed"

    XW = torch.randn(n, 2, device="cuda")
    got = g2.aggregate(2, x=XW).double().sum(dim=0).cpu().numpy()
    want2 = indeg @ oracle.tf32(XW.cpu().numpy()).astype(np.float64)
    print(f"narrow F=2: checksum rel-L2 {rel_l2(got, want2):.2e}", flush=True)
    assert rel_l2(got, want2) <= TOL, "narrow"
    dY = torch.randn(n, 2, device="cuda")
    dX = swtcf.bcsc_transpose_spmm(g2.bwd, dY)
    got = dX[:n].double().sum(dim=0).cpu().numpy()
    wantT = outdeg @ dY.cpu().numpy().astype(np.float64)
    print(f"narrow transpose F=2: checksum rel-L2 {rel_l2(got, wantT):.2e}", flush=True)
    assert rel_l2(got, wantT) <= TOL, "narrow transpose"


def test_fullsize_config3_swtcf(gpu, oracle):
    """convertCOOToSWTCF and the SWTCF SpMM on the config-3 graph (114M
    edges, unit values; F = 128 for time): every edge is exactly one tile
    bit, the product passes the checksum, and it equals the BCSR gather's
    element by element.  X holds TF32 values already, so the SWTCF path's
    per-tile choice between TF32 and fp32 inputs does not change it."""
    from tcc_amd import swtcf
    from tcc_amd.graphs import CONFIGS, make_graph

    n = CONFIGS[3]["n"]
    F = 128
    rows, cols, _ = make_graph(3, device="cuda")
    r32 = rows.to(torch.int32).contiguous()
    c32 = cols.to(torch.int32).contiguous()
    nnz = r32.numel()
    del rows
    print(f"config 3 SWTCF: n={n} nnz={nnz} F={F}", flush=True)
    m = swtcf.DeviceSWTCFMatrix(n, n, nnz, 16)
    ws = swtcf.SWTCFConvertWorkspace(nnz, n, 16)
    swtcf.convertCOOToSWTCF(r32, c32, nnz, m, ws)
    assert ws.device_error() == 0
    h = m.to_host()
    bits = int(np.unpackbits(h["tileLocalBit"].view(np.uint8)).sum())
    print(f"tiles {h['numTiles']}, tile bits {bits}", flush=True)
    assert bits == nnz
    assert np.all(np.diff(h["colWindowOffset"].astype(np.int64)) >= 0)

    X = oracle.tf32(np.random.default_rng(33).standard_normal((n, F)).astype(np.float32))
    Xd = torch.from_numpy(X).cuda()
    Ys = torch.zeros(n, F, device="cuda")
    swtcf.swtcf_spmm(m, Xd, Ys, 12)
    indeg = np.bincount(c32.cpu().numpy().astype(np.int64), minlength=n).astype(np.float64)
    want = indeg @ X.astype(np.float64)
    got = Ys.double().sum(dim=0).cpu().numpy()
    print(f"SWTCF checksum rel-L2 {rel_l2(got, want):.2e}", flush=True)
    assert rel_l2(got, want) <= TOL
    A = swtcf.coo_to_bcsr(r32, c32, None, n, n)
    Yb = swtcf.bcsr_spmm(A, Xd)[:n]
    d = ((Ys.double() - Yb.double()).norm() / Yb.double().norm()).item()
    print(f"SWTCF against the BCSR gather: rel-L2 {d:.2e}", flush=True)
    assert d <= 1e-6
