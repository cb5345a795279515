"""GPU parity of the SpMM kernels against the CPU oracle, through the C-ABI.

Tolerance: rel-L2 <= 1e-3 against the fp64 oracle on TF32-rounded inputs
(the acceptance bound), and a tighter 1e-5 regression bound: the kernels
round exactly the inputs the oracle rounds, so only fp32 summation order
separates them.  The reference's own known-answer test
(src/swtcf_spmm_main.cu:33-112) is checked with its own tolerances.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

REL_L2 = 1e-3
REL_L2_TIGHT = 1e-5


def rel_l2(y, ref):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(y - ref) / (den if den > 0 else 1.0))


def assert_close(y, ref, tight=True):
    e = rel_l2(y, ref)
    assert e <= REL_L2, e
    if tight:
        assert e <= REL_L2_TIGHT, e


def random_coo(nd, ns, nnz, seed):
    rng = np.random.default_rng(seed)
    keys = np.sort(rng.choice(nd * ns, size=nnz, replace=False))
    return (keys // ns).astype(np.uint32), (keys % ns).astype(np.uint32)


def dev_u32(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).cuda()


def build_swtcf(dst, src, rows, cols, S=16):
    from tcc_amd import swtcf

    m = swtcf.DeviceSWTCFMatrix(rows, cols, dst.size, S)
    ws = swtcf.SWTCFConvertWorkspace(dst.size, cols, S)
    swtcf.convertCOOToSWTCF(dev_u32(dst), dev_u32(src), dst.size, m, ws)
    assert ws.device_error() == 0
    return m


# ------------------------------------------------------------------ SWTCF
@pytest.mark.parametrize("tc", [12, 65])
def test_swtcf_kat_reference_tolerances(gpu, oracle, tc):
    """launchSWTCFSpMM with the reference's closed-form X and its tolerances."""
    from tcc_amd import swtcf

    dst, src = random_coo(900, 1500, 20000, 1)
    m = build_swtcf(dst, src, 900, 1500)
    X = torch.from_numpy(oracle.kat_fill_x(1500, 128)).cuda()
    Y = torch.zeros((900, 128), device="cuda")
    swtcf.launchSWTCFSpMM(m, X, Y, tc)
    K = oracle.kat_expected(dst, src, 900, 128)
    atol, rtol = (2e-4, 1e-4) if tc > 64 else (1e-2, 1e-2)
    err = np.abs(Y.cpu().numpy() - K)
    assert np.all(err <= atol + rtol * np.abs(K))


@pytest.mark.parametrize("F", [1, 32, 100, 128, 200])
@pytest.mark.parametrize("tc", [0, 12, 65])
def test_swtcf_spmm_vs_oracle(gpu, oracle, F, tc):
    from tcc_amd import swtcf

    dst, src = random_coo(700, 1100, 15000, 2)
    # a dense block so both threshold branches run
    dd = np.repeat(np.arange(8, dtype=np.uint32), 8)
    ss = np.tile(np.arange(16, 24, dtype=np.uint32), 8)
    keys = np.unique(np.concatenate([dst.astype(np.int64) * 1100 + src, dd.astype(np.int64) * 1100 + ss]))
    dst, src = (keys // 1100).astype(np.uint32), (keys % 1100).astype(np.uint32)
    m = build_swtcf(dst, src, 700, 1100)
    X = np.random.default_rng(3).standard_normal((1100, F)).astype(np.float32)
    Y0 = np.random.default_rng(4).standard_normal((700, F)).astype(np.float32)  # Y += A X
    Y = torch.from_numpy(Y0.copy()).cuda()
    swtcf.swtcf_spmm(m, torch.from_numpy(X).cuda(), Y, tc)
    ref = oracle.swtcf_convert(dst, src, 700, 1100, 16)
    want = oracle.swtcf_spmm(ref, X, tc=tc, rows=700, Y=Y0.astype(np.float64))
    assert_close(Y.cpu().numpy(), want)


@pytest.mark.parametrize("S", [1, 3, 32])
def test_swtcf_spmm_super_window_sizes_skewed(gpu, oracle, S):
    """Super-window sizes other than 16 (1 window per workgroup, 3, and two
    windows per wave at 32) on an R-MAT graph whose hub windows hold many
    tiles (several tile groups per window) and many repeated rows."""
    from tcc_amd import swtcf
    from tcc_amd.graphs import rmat_graph

    n, F = 3000, 48
    rows, cols = rmat_graph(n, 60_000, 21)
    dst, src = rows.numpy().astype(np.uint32), cols.numpy().astype(np.uint32)
    m = build_swtcf(dst, src, n, n, S=S)
    X = np.random.default_rng(5).standard_normal((n, F)).astype(np.float32)
    Y = torch.zeros((n, F), device="cuda")
    swtcf.swtcf_spmm(m, torch.from_numpy(X).cuda(), Y, 12)
    ref = oracle.swtcf_convert(dst, src, n, n, S)
    assert int(np.max(np.diff(ref["colWindowOffset"]))) > 16  # windows with several tile groups
    want = oracle.swtcf_spmm(ref, X, tc=12, rows=n)
    assert_close(Y.cpu().numpy(), want)


@pytest.mark.parametrize("F", [64, 128, 200])
def test_swtcf_hub_windows_split_across_waves(gpu, oracle, F):
    """Super-windows whose windows are unbalanced (one source column with
    ~3000 destinations, hundreds of tiles in one window) have their tiles cut
    into equal ranges across the waves of several parts, cuts inside the hub
    window and snapped to short windows' boundaries."""
    from tcc_amd import swtcf

    nr, nc = 6000, 700
    rng = np.random.default_rng(31)
    keys = set(rng.choice(nr * nc, size=20000, replace=False).tolist())
    for c in (5, 300, 301):  # hub sources: long windows 0 and 37
        keys.update(r * nc + c for r in rng.choice(nr, size=3000, replace=False).tolist())
    k = np.array(sorted(keys), np.int64)
    dst, src = (k // nc).astype(np.uint32), (k % nc).astype(np.uint32)
    m = build_swtcf(dst, src, nr, nc)
    ref = oracle.swtcf_convert(dst, src, nr, nc, 16)
    lens = np.diff(ref["colWindowOffset"])
    assert lens.max() > 8 * lens.mean()  # the split path
    X = np.random.default_rng(32).standard_normal((nc, F)).astype(np.float32)
    Y0 = np.random.default_rng(33).standard_normal((nr, F)).astype(np.float32)
    Y = torch.from_numpy(Y0.copy()).cuda()
    swtcf.swtcf_spmm(m, torch.from_numpy(X).cuda(), Y, 12)
    want = oracle.swtcf_spmm(ref, X, tc=12, rows=nr, Y=Y0.astype(np.float64))
    assert_close(Y.cpu().numpy(), want)


@pytest.mark.parametrize("F", [1, 48, 100, 200])
@pytest.mark.parametrize("mf", [0, 12, 32, 64, 65])
def test_swtcf_spmm_mfma_vs_oracle(gpu, oracle, mf, F):
    """tcc_swtcf_spmm_mfma: tiles of >= max(mf, tc) entries on fp32 MFMA,
    two per instruction, on a graph with dense 8x8 blocks of every density
    (8..64 entries, odd and even counts per window so that a tile is left
    without a partner), an R-MAT part (repeat-cache rows, long windows) and
    Y += A X; against the oracle's TF32 numerics for those tiles."""
    from tcc_amd import swtcf
    from tcc_amd.graphs import rmat_graph

    n = 2000
    rows, cols = rmat_graph(n, 30_000, 41)
    keys = set((rows.numpy().astype(np.int64) * n + cols.numpy()).tolist())
    rng = np.random.default_rng(42)
    for b, k in enumerate([8, 16, 24, 32, 40, 48, 56, 64, 64, 33, 47, 12]):
        r0, c0 = 8 * (10 + b), 8 * (3 + (b % 5))  # several blocks share a window
        for bit in rng.choice(64, size=k, replace=False):
            keys.add((r0 + bit // 8) * n + c0 + bit % 8)
    key = np.array(sorted(keys), np.int64)
    dst, src = (key // n).astype(np.uint32), (key % n).astype(np.uint32)
    m = build_swtcf(dst, src, n, n)
    X = np.random.default_rng(43).standard_normal((n, F)).astype(np.float32)
    Y0 = np.random.default_rng(44).standard_normal((n, F)).astype(np.float32)
    Y = torch.from_numpy(Y0.copy()).cuda()
    swtcf.swtcf_spmm_mfma(m, torch.from_numpy(X).cuda(), Y, 12, mf)
    ref = oracle.swtcf_convert(dst, src, n, n, 16)
    want = oracle.swtcf_spmm(ref, X, tc=12, rows=n, Y=Y0.astype(np.float64))
    assert_close(Y.cpu().numpy(), want)


def test_swtcf_config1(gpu, oracle):
    from tcc_amd import swtcf
    from tcc_amd.graphs import make_features, uniform_graph

    rows, cols = uniform_graph(4096, 16, 1)
    dst, src = rows.numpy().astype(np.uint32), cols.numpy().astype(np.uint32)
    m = build_swtcf(dst, src, 4096, 4096)
    X = make_features(4096, 32, 1, dist="uniform")
    Y = torch.zeros((4096, 32), device="cuda")
    swtcf.swtcf_spmm(m, X.cuda(), Y, 12)
    want = oracle.swtcf_spmm(oracle.swtcf_convert(dst, src, 4096, 4096, 16), X.numpy(), tc=12, rows=4096)
    assert_close(Y.cpu().numpy(), want)


def test_swtcf_quantized(gpu, oracle):
    from tcc_amd import swtcf

    dst, src = random_coo(500, 800, 9000, 5)
    m = build_swtcf(dst, src, 500, 800)
    rng = np.random.default_rng(6)
    n_global = 1000
    q = rng.integers(-128, 128, size=(n_global, 128), dtype=np.int8)
    scales = rng.uniform(0.001, 0.1, n_global).astype(np.float32)
    srcGlobal = rng.choice(n_global, size=800, replace=False).astype(np.uint32)
    Y = torch.zeros((500, 128), device="cuda")
    swtcf.launchSWTCFSpMMQuantized(m, torch.from_numpy(q).cuda(), torch.from_numpy(scales).cuda(),
                                   dev_u32(srcGlobal), Y, 12)
    Xdeq = q[srcGlobal].astype(np.float32) * scales[srcGlobal][:, None]  # src/swtcf_spmm.cu:317-323
    want = oracle.swtcf_spmm(oracle.swtcf_convert(dst, src, 500, 800, 16), Xdeq, tc=12, rows=500)
    assert_close(Y.cpu().numpy(), want)


# ------------------------------------------------------------------ blocks
def csr_of(dst, src, n, vals=None):
    order = np.lexsort((src, dst))
    rowptr = np.zeros(n + 1, np.int64)
    rowptr[1:] = np.cumsum(np.bincount(dst, minlength=n))
    return rowptr, src[order], None if vals is None else vals[order]


def csc_of(dst, src, ncols, vals=None):
    order = np.lexsort((dst, src))
    colptr = np.zeros(ncols + 1, np.int64)
    colptr[1:] = np.cumsum(np.bincount(src, minlength=ncols))
    return colptr, dst[order], None if vals is None else vals[order]


@pytest.mark.parametrize("values", [False, True])
def test_coo_to_bcsr_bcsc_bit_exact(gpu, oracle, values):
    from tcc_amd import swtcf

    nr, nc = 1003, 1501
    dst, src = random_coo(nr, nc, 25000, 7)
    vals = np.random.default_rng(8).uniform(0.1, 1, dst.size).astype(np.float32) if values else None
    perm = np.random.default_rng(9).permutation(dst.size)  # unsorted input
    tv = None if vals is None else torch.from_numpy(vals[perm]).cuda()
    A = swtcf.coo_to_bcsr(dev_u32(dst[perm]), dev_u32(src[perm]), tv, nr, nc).to_host()
    rowptr, colind, v = csr_of(dst, src, nr, vals)
    want = oracle.bcsr_build(nr, nc, rowptr, colind, v)
    for k in ("rowWindowOffset", "tcOffset", "sparseA2B", "tcLocalBit"):
        assert np.array_equal(A[k], want[k][:A[k].size]), k
    assert A["num_TCBlocks"] == want["num_TCBlocks"]
    if values:
        assert np.array_equal(A["data"], want["data"])
    B = swtcf.coo_to_bcsc(dev_u32(dst[perm]), dev_u32(src[perm]), tv, nr, nc).to_host()
    colptr, rowind, cv = csc_of(dst, src, nc, vals)
    wantc = oracle.bcsc_build(nr, nc, colptr, rowind, cv)
    for k in ("colWindowOffset", "tcOffset", "sparseA2C", "tcLocalBit"):
        assert np.array_equal(B[k], wantc[k][:B[k].size]), k
    if values:
        assert np.array_equal(B["data"], wantc["data"])


@pytest.mark.parametrize("F", [1, 2, 3, 5, 8, 13, 16, 17, 32, 100, 128, 256, 602])
@pytest.mark.parametrize("values", [False, True])
def test_bcsr_bcsc_spmm_vs_oracle(gpu, oracle, F, values):
    """F <= 16 runs the narrow gather (8 blocks per wave step; F = 3, 13 take
    the element-wise row loads, 8 and 16 the vector ones), F >= 17 the
    feature-chunk gather."""
    from tcc_amd import swtcf

    nr, nc = 777, 901
    dst, src = random_coo(nr, nc, 12000, 10 + F)
    vals = np.random.default_rng(11).uniform(-1, 1, dst.size).astype(np.float32) if values else None
    X = np.random.default_rng(12).standard_normal((nc, F)).astype(np.float32)
    Xd = torch.from_numpy(X).cuda()
    rowptr, colind, v = csr_of(dst, src, nr, vals)
    want = oracle.csr_spmm(rowptr, colind, v, X, use_tf32=True)
    tv = None if vals is None else torch.from_numpy(vals).cuda()
    A = swtcf.coo_to_bcsr(dev_u32(dst), dev_u32(src), tv, nr, nc)
    Y = swtcf.bcsr_spmm(A, Xd)
    assert_close(Y.cpu().numpy()[:nr], want)
    assert np.all(Y.cpu().numpy()[nr:] == 0)  # padding rows of the last window
    # accumulate form
    Y2 = swtcf.bcsr_spmm(A, Xd, Y.clone(), accumulate=True)
    assert_close(Y2.cpu().numpy()[:nr], 2 * want)
    Bc = swtcf.coo_to_bcsc(dev_u32(dst), dev_u32(src), tv, nr, nc)
    Yc = torch.zeros((nr, F), device="cuda")
    swtcf.bcsc_spmm(Bc, Xd, Yc)
    assert_close(Yc.cpu().numpy(), want)
    # backward: A^T dY via the BCSC as a gather
    dY = np.random.default_rng(13).standard_normal((nr, F)).astype(np.float32)
    colptr = np.zeros(nc + 1, np.int64)
    order = np.lexsort((dst, src))
    colptr[1:] = np.cumsum(np.bincount(src, minlength=nc))
    wantT = oracle.csr_spmm(colptr, dst[order], None if vals is None else vals[order], dY, use_tf32=False)
    dX = swtcf.bcsc_transpose_spmm(Bc, torch.from_numpy(dY).cuda())
    assert_close(dX.cpu().numpy()[:nc], wantT)


def test_oracle_built_blocks_consumed_identically(gpu, oracle):
    """Kernels take any valid BCSR/BCSC (here the oracle's, uploaded as-is)."""
    from tcc_amd import swtcf

    nr, nc, F = 500, 640, 64
    dst, src = random_coo(nr, nc, 7000, 14)
    vals = np.random.default_rng(15).uniform(-1, 1, dst.size).astype(np.float32)
    rowptr, colind, v = csr_of(dst, src, nr, vals)
    d = oracle.bcsr_build(nr, nc, rowptr, colind, v)
    X = np.random.default_rng(16).standard_normal((nc, F)).astype(np.float32)
    Y = swtcf.bcsr_spmm(swtcf.host_to_bcsr(d, use_data=True), torch.from_numpy(X).cuda())
    assert_close(Y.cpu().numpy(), oracle.bcsr_spmm(d, X, use_data=True))


def test_spmm_cnic_forward_hot_cold_split(gpu, oracle):
    """denseC = A_bcsr X + A_bcsc X (spmm_launcher.cu:203-271) with A split
    into the edges of hot and cold sources."""
    from tcc_amd import swtcf

    nr = nc = 1200
    F = 128
    dst, src = random_coo(nr, nc, 20000, 17)
    hot = np.random.default_rng(18).random(nc) < 0.3
    h = hot[src]
    A = swtcf.coo_to_bcsr(dev_u32(dst[h]), dev_u32(src[h]), None, nr, nc)
    B = swtcf.coo_to_bcsc(dev_u32(dst[~h]), dev_u32(src[~h]), None, nr, nc)
    X = np.random.default_rng(19).standard_normal((nc, F)).astype(np.float32)
    denseC = torch.full(((A.view.num_rowWindows + 1) * 8, F), 7.0, device="cuda")  # garbage in
    swtcf.spmm_cnic_forward(A, B, torch.from_numpy(X).cuda(), denseC)
    rowptr, colind, _ = csr_of(dst, src, nr)
    want = oracle.csr_spmm(rowptr, colind, None, X, use_tf32=True)
    C = denseC.cpu().numpy()
    assert_close(C[:nr], want)
    assert np.all(C[nr:] == 0)


def test_mixed_hot_cold_feature_source(gpu, oracle):
    """First-layer form: hot rows from an HBM cache, cold rows zero-copy from
    mapped pinned host memory (spmm_kernel.cu:129-153)."""
    from tcc_amd import swtcf
    from tcc_amd.hostmem import PinnedArray

    nr = nc = 1000
    F = 100
    dst, src = random_coo(nr, nc, 15000, 20)
    rng = np.random.default_rng(21)
    feats = rng.standard_normal((nc, F)).astype(np.float32)  # global feature table, ids = identity
    hot_ids = np.sort(rng.choice(nc, size=nc // 5, replace=False))
    csm = np.full(nc, -1, np.int32)
    csm[hot_ids] = np.arange(hot_ids.size, dtype=np.int32)
    id_map = np.arange(nc, dtype=np.int32)
    id_map[7] = -1  # a column with no feature row reads zeros
    csm[7] = -1
    hot_cache = torch.from_numpy(feats[hot_ids]).cuda()
    cpu = PinnedArray((nc, F))
    cpu.array[:] = feats
    ptrs = torch.tensor([hot_cache.data_ptr()], dtype=torch.int64, device="cuda")
    id_map_d = torch.from_numpy(id_map).cuda()
    csm_d = torch.from_numpy(csm).cuda()
    # the handle keeps id_map_d / csm_d / ptrs alive for the launch below
    src_desc = swtcf.feature_source(id_map_d, csm_d, ptrs, hot_ids.size, cpu.device_ptr, nc * F)
    hot_mask = csm[src] >= 0
    A = swtcf.coo_to_bcsr(dev_u32(dst[hot_mask]), dev_u32(src[hot_mask]), None, nr, nc)
    B = swtcf.coo_to_bcsc(dev_u32(dst[~hot_mask]), dev_u32(src[~hot_mask]), None, nr, nc)
    denseC = torch.empty(((A.view.num_rowWindows + 1) * 8, F), device="cuda")
    swtcf.spmm_cnic_forward_mixed(A, B, src_desc, denseC, F)
    Xres = oracle.resolve_features(id_map, csm, feats[hot_ids], hot_ids.size, feats, F)
    rowptr, colind, _ = csr_of(dst, src, nr)
    want = oracle.csr_spmm(rowptr, colind, None, Xres, use_tf32=True)
    assert_close(denseC.cpu().numpy()[:nr], want)
    torch.cuda.synchronize()
    cpu.free()


@pytest.mark.parametrize("packed", [False, True])
def test_mixed_refused_lookups_read_zeros_and_set_the_error(gpu, oracle, packed):
    """Lookups outside their table (a cache index past the pointer table, a
    host row past cpu_feature_len) are refused by the kernels' own bounds
    checks: they read zeros and write TCC_DEVERR_FEATURE_INDEX to the
    source's error word; a source without bad entries leaves it at 0."""
    from tcc_amd import swtcf
    from tcc_amd.hostmem import PinnedArray

    nr = nc = 600
    F = 64
    dst, src = random_coo(nr, nc, 8000, 31)
    rng = np.random.default_rng(32)
    feats = rng.standard_normal((nc, F)).astype(np.float32)
    hot_ids = np.sort(rng.choice(nc, size=nc // 4, replace=False))
    csm = np.full(nc, -1, np.int32)
    csm[hot_ids] = np.arange(hot_ids.size, dtype=np.int32)
    id_map = np.arange(nc, dtype=np.int32)
    cold = np.setdiff1d(np.arange(nc), hot_ids)
    bad_cache = int(hot_ids[3])  # cache index cap + 3: pointer-table entry 1 of 1
    bad_host = int(cold[5])      # host row past the table's last row
    csm[bad_cache] = hot_ids.size + 3
    cpu_rows = nc                # cpu_feature_len covers rows 0 .. nc-1
    id_map[bad_host] = nc
    if packed:
        stride = packed_stride_host(F)
        hot_cache = swtcf.tf32_pack(torch.from_numpy(feats[hot_ids]).cuda())
        cpu = PinnedArray((nc * stride,), np.uint8)
        cpu.array[:] = swtcf.tf32_pack(torch.from_numpy(feats).cuda()).cpu().numpy()[: nc * stride]
        fmt = swtcf.ROWS_TF32_PACKED
    else:
        hot_cache = torch.from_numpy(feats[hot_ids]).cuda()
        cpu = PinnedArray((nc, F))
        cpu.array[:] = feats
        fmt = swtcf.ROWS_FP32
    ptrs = torch.tensor([hot_cache.data_ptr()], dtype=torch.int64, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    print(f"refused lookups: packed={packed} bad cache column {bad_cache}, bad host column {bad_host}", flush=True)
    src_desc = swtcf.feature_source(torch.from_numpy(id_map).cuda(), torch.from_numpy(csm).cuda(), ptrs,
                                    hot_ids.size, cpu.device_ptr, cpu_rows * F, row_format=fmt, device_error=err)
    hot_mask = csm[src] >= 0
    A = swtcf.coo_to_bcsr(dev_u32(dst[hot_mask]), dev_u32(src[hot_mask]), None, nr, nc)
    B = swtcf.coo_to_bcsc(dev_u32(dst[~hot_mask]), dev_u32(src[~hot_mask]), None, nr, nc)
    assert np.any(src == bad_cache) and np.any(src == bad_host)
    denseC = torch.empty(((A.view.num_rowWindows + 1) * 8, F), device="cuda")
    swtcf.spmm_cnic_forward_mixed(A, B, src_desc, denseC, F)
    X = feats.copy()
    X[bad_cache] = 0.0
    X[bad_host] = 0.0
    rowptr, colind, _ = csr_of(dst, src, nr)
    assert_close(denseC.cpu().numpy()[:nr], oracle.csr_spmm(rowptr, colind, None, X, use_tf32=True))
    assert int(err.item()) == swtcf.DEVERR_FEATURE_INDEX
    # the same matrices over a valid source: no error
    csm_ok = np.full(nc, -1, np.int32)
    csm_ok[hot_ids] = np.arange(hot_ids.size, dtype=np.int32)
    err.zero_()
    ok = swtcf.feature_source(torch.from_numpy(np.arange(nc, dtype=np.int32)).cuda(), torch.from_numpy(csm_ok).cuda(),
                              ptrs, hot_ids.size, cpu.device_ptr, nc * F, row_format=fmt, device_error=err)
    swtcf.spmm_cnic_forward_mixed(A, B, ok, denseC, F)
    assert_close(denseC.cpu().numpy()[:nr], oracle.csr_spmm(rowptr, colind, None, feats, use_tf32=True))
    assert int(err.item()) == 0
    torch.cuda.synchronize()
    cpu.free()


@pytest.mark.parametrize("F,vals_hot,vals_cold,K", [(37, True, True, 0), (100, True, False, 3), (100, False, True, 0),
                                                    (256, True, True, 5), (100, False, False, 2)])
def test_mixed_forward_values_widths_units(gpu, oracle, F, vals_hot, vals_cold, K):
    """The first-layer forward in one launch (hot gather and cold scatter
    interleaved, both adding into a zeroed denseC): every value combination,
    V = 1, 2, 4 and unit sizes that split windows, against the CSR oracle on
    the resolved features."""
    from tcc_amd import swtcf
    from tcc_amd.hostmem import PinnedArray

    nr = nc = 1500
    dst, src = random_coo(nr, nc, 30000, 40 + F)
    rng = np.random.default_rng(41 + F)
    vals = rng.uniform(0.5, 1.5, dst.size).astype(np.float32)
    feats = rng.standard_normal((nc, F)).astype(np.float32)
    hot_ids = np.sort(rng.choice(nc, size=nc // 4, replace=False))
    csm = np.full(nc, -1, np.int32)
    csm[hot_ids] = np.arange(hot_ids.size, dtype=np.int32)
    id_map = np.arange(nc, dtype=np.int32)
    hot_cache = torch.from_numpy(feats[hot_ids]).cuda()
    cpu = PinnedArray((nc, F))
    cpu.array[:] = feats
    ptrs = torch.tensor([hot_cache.data_ptr()], dtype=torch.int64, device="cuda")
    id_map_d = torch.from_numpy(id_map).cuda()
    csm_d = torch.from_numpy(csm).cuda()
    src_desc = swtcf.feature_source(id_map_d, csm_d, ptrs, hot_ids.size, cpu.device_ptr, nc * F)
    h = csm[src] >= 0
    vh = torch.from_numpy(vals[h]).cuda() if vals_hot else None
    vc = torch.from_numpy(vals[~h]).cuda() if vals_cold else None
    A = swtcf.coo_to_bcsr(dev_u32(dst[h]), dev_u32(src[h]), vh, nr, nc)
    B = swtcf.coo_to_bcsc(dev_u32(dst[~h]), dev_u32(src[~h]), vc, nr, nc)
    A.set_unit_blocks(K)
    B.set_unit_blocks(K)
    denseC = torch.full(((A.view.num_rowWindows + 1) * 8, F), 3.0, device="cuda")  # garbage in
    swtcf.spmm_cnic_forward_mixed(A, B, src_desc, denseC, F)
    used = np.where(h, vals if vals_hot else 1.0, vals if vals_cold else 1.0).astype(np.float32)
    rowptr, colind, v = csr_of(dst, src, nr, used)
    want = oracle.csr_spmm(rowptr, colind, v, feats, use_tf32=True)
    C = denseC.cpu().numpy()
    assert_close(C[:nr], want)
    assert np.all(C[nr:] == 0)
    torch.cuda.synchronize()
    cpu.free()


@pytest.mark.parametrize("case", ["all_cold", "all_hot", "many_units", "many_units_packed"])
def test_mixed_forward_extremes(gpu, oracle, case):
    """The one-launch forward with no hot edges (no gather units), with no
    cold edges (no scatter), and with more scatter units than its persistent
    waves (K = 1 over ~9k cold blocks, so each scatter wave walks several)."""
    from tcc_amd import swtcf
    from tcc_amd.hostmem import PinnedArray

    big = case.startswith("many_units")
    nr = nc = 6000 if big else 1200
    F = 100
    dst, src = random_coo(nr, nc, 120000 if big else 20000, 71)
    rng = np.random.default_rng(72)
    feats = rng.standard_normal((nc, F)).astype(np.float32)
    frac = {"all_cold": 0.0, "all_hot": 1.0}.get(case, 0.2)
    hot_ids = np.sort(rng.choice(nc, size=int(nc * frac), replace=False))
    csm = np.full(nc, -1, np.int32)
    csm[hot_ids] = np.arange(hot_ids.size, dtype=np.int32)
    id_map = np.arange(nc, dtype=np.int32)
    packed = case == "many_units_packed"
    if packed:
        hot_cache = swtcf.tf32_pack(torch.from_numpy(feats[hot_ids]).cuda()) if hot_ids.size else None
        row_bytes = packed_stride_host(F)
        cpu = PinnedArray((nc * row_bytes,), np.uint8)
        cpu.array[:] = swtcf.tf32_pack(torch.from_numpy(feats).cuda()).cpu().numpy()[: nc * row_bytes]
        fmt = swtcf.ROWS_TF32_PACKED
    else:
        hot_cache = torch.from_numpy(feats[hot_ids]).cuda() if hot_ids.size else None
        cpu = PinnedArray((nc, F))
        cpu.array[:] = feats
        fmt = swtcf.ROWS_FP32
    keep = hot_cache if hot_cache is not None else torch.zeros(16, device="cuda")
    ptrs = torch.tensor([keep.data_ptr()], dtype=torch.int64, device="cuda")
    id_map_d = torch.from_numpy(id_map).cuda()
    csm_d = torch.from_numpy(csm).cuda()
    src_desc = swtcf.feature_source(id_map_d, csm_d, ptrs, max(hot_ids.size, 1), cpu.device_ptr, nc * F,
                                    row_format=fmt)
    h = csm[src] >= 0
    A = swtcf.coo_to_bcsr(dev_u32(dst[h]), dev_u32(src[h]), None, nr, nc)
    B = swtcf.coo_to_bcsc(dev_u32(dst[~h]), dev_u32(src[~h]), None, nr, nc)
    if big:
        B.set_unit_blocks(1)
        assert B.view.num_TCBlocks > 4096
    denseC = torch.full(((A.view.num_rowWindows + 1) * 8, F), 3.0, device="cuda")  # garbage in
    swtcf.spmm_cnic_forward_mixed(A, B, src_desc, denseC, F)
    rowptr, colind, _ = csr_of(dst, src, nr)
    want = oracle.csr_spmm(rowptr, colind, None, feats, use_tf32=True)
    C = denseC.cpu().numpy()
    assert_close(C[:nr], want)
    assert np.all(C[nr:] == 0)
    torch.cuda.synchronize()
    cpu.free()


@pytest.mark.parametrize("F,values,K", [(37, True, 0), (100, False, 3), (256, True, 0), (301, True, 2),
                                         (602, False, 0)])
def test_mixed_forward_packed_rows(gpu, oracle, F, values, K):
    """A feature source of packed TF32 rows (hot cache and host table in the
    tcc_tf32_pack layout): the one-launch forward and the hot gather alone
    give the oracle's TF32 product, as the fp32 rows do (F = 301, 602: 4-wide
    chunks with a partial last lane)."""
    from tcc_amd import swtcf
    from tcc_amd.hostmem import PinnedArray

    nr = nc = 1300
    dst, src = random_coo(nr, nc, 26000, 70 + F)
    rng = np.random.default_rng(71 + F)
    vals = rng.uniform(0.5, 1.5, dst.size).astype(np.float32)
    feats = rng.standard_normal((nc, F)).astype(np.float32)
    hot_ids = np.sort(rng.choice(nc, size=nc // 3, replace=False))
    csm = np.full(nc, -1, np.int32)
    csm[hot_ids] = np.arange(hot_ids.size, dtype=np.int32)
    id_map = np.arange(nc, dtype=np.int32)
    hot_cache = swtcf.tf32_pack(torch.from_numpy(feats[hot_ids]).cuda())
    rows = swtcf.tf32_pack(torch.from_numpy(feats).cuda()).cpu().numpy()
    cpu = PinnedArray((rows.size,), dtype=np.uint8)
    cpu.array[:] = rows
    ptrs = torch.tensor([hot_cache.data_ptr()], dtype=torch.int64, device="cuda")
    id_map_d = torch.from_numpy(id_map).cuda()
    csm_d = torch.from_numpy(csm).cuda()
    src_desc = swtcf.feature_source(id_map_d, csm_d, ptrs, hot_ids.size, cpu.device_ptr, nc * F,
                                    swtcf.ROWS_TF32_PACKED)
    h = csm[src] >= 0
    vh = torch.from_numpy(vals[h]).cuda() if values else None
    vc = torch.from_numpy(vals[~h]).cuda() if values else None
    A = swtcf.coo_to_bcsr(dev_u32(dst[h]), dev_u32(src[h]), vh, nr, nc)
    B = swtcf.coo_to_bcsc(dev_u32(dst[~h]), dev_u32(src[~h]), vc, nr, nc)
    A.set_unit_blocks(K)
    B.set_unit_blocks(K)
    denseC = torch.full(((A.view.num_rowWindows + 1) * 8, F), 3.0, device="cuda")
    swtcf.spmm_cnic_forward_mixed(A, B, src_desc, denseC, F)
    used = vals if values else None
    rowptr, colind, v = csr_of(dst, src, nr, used)
    want = oracle.csr_spmm(rowptr, colind, v, feats, use_tf32=True)
    C = denseC.cpu().numpy()
    assert_close(C[:nr], want)
    assert np.all(C[nr:] == 0)
    # the hot gather alone (tcc_bcsr_spmm_mixed) over the hot edges
    Yh = swtcf.bcsr_spmm_mixed(A, src_desc, torch.empty((A.view.num_rowWindows * 8, F), device="cuda"), F)
    rp, ci, vv = csr_of(dst[h], src[h], nr, vals[h] if values else None)
    assert_close(Yh.cpu().numpy()[:nr], oracle.csr_spmm(rp, ci, vv, feats, use_tf32=True))
    torch.cuda.synchronize()
    cpu.free()


# ------------------------------------------------------------------ units of work
def skewed_coo(nr, nc, seed):
    """A few dense hub rows and hub columns over a sparse background, with
    bands of empty row/column windows inside and at the end."""
    rng = np.random.default_rng(seed)
    keys = set(rng.choice(nr * nc, size=6000, replace=False).tolist())
    for r in (3, 4, 500):  # hub rows -> long BCSR windows
        keys.update(r * nc + c for c in rng.choice(nc, size=nc // 2, replace=False).tolist())
    for c in (7, 600):  # hub columns -> long BCSC windows
        keys.update(r * nc + c for r in rng.choice(nr, size=nr // 2, replace=False).tolist())
    k = np.array(sorted(keys), np.int64)
    r, c = k // nc, k % nc
    keep = ~(((r >= 200) & (r < 264)) | (r >= 600) | ((c >= 300) & (c < 340)) | (c >= 880))
    return r[keep].astype(np.uint32), c[keep].astype(np.uint32)


@pytest.mark.parametrize("unit_blocks", [0, 1, 2, 3, 5, 8, 64])
@pytest.mark.parametrize("F", [2, 7, 13, 64, 128, 256, 602])
def test_units_split_windows(gpu, oracle, unit_blocks, F):
    """Units of K consecutive blocks cut windows anywhere (empty windows
    included); windows shared by several units add their partial sums
    atomically into pre-zeroed rows.  Every K gives the oracle's product, for
    the BCSR gather (= and +=), the BCSC scatter and the BCSC^T gather."""
    from tcc_amd import swtcf

    nr, nc = 640, 900
    dst, src = skewed_coo(nr, nc, 30 + F)
    vals = np.random.default_rng(31).uniform(-1, 1, dst.size).astype(np.float32)
    X = np.random.default_rng(32).standard_normal((nc, F)).astype(np.float32)
    Xd = torch.from_numpy(X).cuda()
    rowptr, colind, v = csr_of(dst, src, nr, vals)
    want = oracle.csr_spmm(rowptr, colind, v, X, use_tf32=True)
    A = swtcf.coo_to_bcsr(dev_u32(dst), dev_u32(src), torch.from_numpy(vals).cuda(), nr, nc)
    A.set_unit_blocks(unit_blocks)
    Y = swtcf.bcsr_spmm(A, Xd, torch.full((A.view.num_rowWindows * 8, F), 9.0, device="cuda"))
    assert_close(Y.cpu().numpy()[:nr], want)
    Y2 = swtcf.bcsr_spmm(A, Xd, Y.clone(), accumulate=True)
    assert_close(Y2.cpu().numpy()[:nr], 2 * want)
    B = swtcf.coo_to_bcsc(dev_u32(dst), dev_u32(src), torch.from_numpy(vals).cuda(), nr, nc)
    B.set_unit_blocks(unit_blocks)
    Yc = torch.zeros((nr, F), device="cuda")
    swtcf.bcsc_spmm(B, Xd, Yc)
    assert_close(Yc.cpu().numpy(), want)
    dY = np.random.default_rng(33).standard_normal((nr, F)).astype(np.float32)
    order = np.lexsort((dst, src))
    colptr = np.zeros(nc + 1, np.int64)
    colptr[1:] = np.cumsum(np.bincount(src, minlength=nc))
    wantT = oracle.csr_spmm(colptr, dst[order], vals[order], dY, use_tf32=False)
    dX = swtcf.bcsc_transpose_spmm(B, torch.from_numpy(dY).cuda(),
                                   torch.full((B.view.num_colWindows * 8, F), 5.0, device="cuda"))
    assert_close(dX.cpu().numpy()[:nc], wantT)


def test_empty_coo_builders(gpu):
    """No edges: both builders give empty windows and no blocks, and both
    products leave zeros (BCSR =) or Y unchanged (BCSC +=)."""
    from tcc_amd import swtcf

    e = torch.empty(0, dtype=torch.int32, device="cuda")
    A = swtcf.coo_to_bcsr(e, e, None, 20, 30)
    B = swtcf.coo_to_bcsc(e, e, None, 20, 30)
    assert A.view.num_TCBlocks == 0 and A.view.num_rowWindows == 3
    assert B.view.num_TCBlocks == 0 and B.view.num_colWindows == 4
    hb = B.to_host()
    assert not hb["colWindowOffset"].any() and hb["colWindowOffset"].size == 5
    X = torch.randn((30, 16), device="cuda")
    assert torch.count_nonzero(swtcf.bcsr_spmm(A, X, torch.full((24, 16), 3.0, device="cuda"))).item() == 0
    Y = torch.full((20, 16), 3.0, device="cuda")
    swtcf.bcsc_spmm(B, X, Y)
    assert bool((Y == 3.0).all())


def test_all_windows_empty(gpu):
    """A BCSR with no blocks writes zeros to every row (and += leaves Y)."""
    from tcc_amd import swtcf

    RW, F = 37, 70
    d = dict(num_rows=RW * 8, num_cols=50, nnz=0, num_TCBlocks=0, num_rowWindows=RW,
             rowWindowOffset=np.zeros(RW + 1, np.uint32), tcOffset=np.zeros(1, np.uint32),
             sparseA2B=np.full(8, 0xFFFFFFFF, np.uint32), tcLocalBit=np.zeros(1, np.uint64),
             data=np.zeros(1, np.float32))
    A = swtcf.host_to_bcsr(d)
    X = torch.randn((50, F), device="cuda")
    Y = swtcf.bcsr_spmm(A, X, torch.full((RW * 8, F), 3.0, device="cuda"))
    assert torch.count_nonzero(Y).item() == 0
    Y = swtcf.bcsr_spmm(A, X, torch.full((RW * 8, F), 3.0, device="cuda"), accumulate=True)
    assert bool((Y == 3.0).all())


def test_unit_sizes_agree_on_rmat(gpu):
    """R-MAT windows of very different lengths: every unit size gives the
    same product (to fp32 reassociation) as the automatic one."""
    from tcc_amd import swtcf
    from tcc_amd.graphs import make_features, rmat_graph, sym_norm_values

    n = 20_000
    rows, cols = rmat_graph(n, 200_000, 5)
    vals = sym_norm_values(rows, cols, n)
    A = swtcf.coo_to_bcsr(rows.to(torch.int32).cuda(), cols.to(torch.int32).cuda(), vals.cuda(), n, n)
    X = make_features(n, 96, 5, device="cuda")
    ref = swtcf.bcsr_spmm(A, X).clone()
    for K in (1, 7, 8, 100, 4096):
        A.set_unit_blocks(K)
        Y = swtcf.bcsr_spmm(A, X)
        assert rel_l2(Y.cpu().numpy(), ref.cpu().numpy()) < 1e-6, K


# ------------------------------------------------------------------ packed TF32 rows
def packed_stride_host(F):
    """Row stride of the packed layout (include/tcc_spmm_cnic.h)."""
    full, tail = divmod(F, 256)
    nbytes = full * 640 + ((2 * tail + (tail + 1) // 2 + 15) // 16 * 16 if tail else 0)
    return (nbytes + 127) // 128 * 128 if F > 256 else nbytes


def unpack_host(buf, rows, F):
    """Independent host reading of the packed layout (include/tcc_spmm_cnic.h):
    chunks of 256 features, each 2n bytes of high halves then the 3 low
    mantissa bits of element pairs; full chunks 640 bytes."""
    stride = packed_stride_host(F)
    b = np.asarray(buf, np.uint8)[: rows * stride].reshape(rows, stride)
    out = np.empty((rows, F), np.uint32)
    for c0 in range(0, F, 256):
        n = min(256, F - c0)
        base = (c0 // 256) * 640
        hi = b[:, base: base + 2 * n].copy().view(np.uint16).astype(np.uint32)
        lo_bytes = b[:, base + 2 * n: base + 2 * n + (n + 1) // 2].astype(np.uint32)
        lo = np.empty((rows, n), np.uint32)
        lo[:, 0::2] = lo_bytes[:, : (n + 1) // 2] & 7
        lo[:, 1::2] = (lo_bytes[:, : n // 2] >> 3) & 7
        out[:, c0: c0 + n] = (hi << 16) | (lo << 13)
    return out


@pytest.mark.parametrize("F", [1, 2, 3, 7, 100, 128, 256, 257, 300, 513, 602])
def test_tf32_pack_is_exact(gpu, oracle, F):
    from tcc_amd import swtcf

    rows = 37
    rng = np.random.default_rng(F)
    with np.errstate(over="ignore"):
        X = (rng.standard_normal((rows, F)) * 10.0 ** rng.integers(-30, 30, (rows, F))).astype(np.float32)
    special = np.array([0x3F801000, 0xBF801000, 0x3F800FFF, 0x3F7FF000, 0x7F7FF000, 0x00001000, 0x80000000,
                        0x00000000, 0x7F800000, 0xFF800000], np.uint32).view(np.float32)
    flat = X.reshape(-1)
    flat[: min(special.size, flat.size)] = special[: flat.size]
    packed = swtcf.tf32_pack(torch.from_numpy(X).cuda())
    got = unpack_host(packed.cpu().numpy(), rows, F)
    want = oracle.tf32(X).view(np.uint32)
    assert np.array_equal(got, want)


def test_tf32_pack_keeps_nan(gpu):
    """NaN stays NaN in the packed rows, also when its payload lies only in
    the 13 low bits that TF32 drops (it unpacks quiet, top 19 bits kept)."""
    from tcc_amd import swtcf

    F = 300
    X = np.random.default_rng(5).standard_normal((3, F)).astype(np.float32)
    nans = np.array([0x7F800001, 0xFF800001, 0x7FC00000, 0x7F801000, 0xFFFFFFFF, 0x7FFFF000], np.uint32)
    X.reshape(-1)[[0, 7, 255, 256, 299, 600]] = nans.view(np.float32)
    got = unpack_host(swtcf.tf32_pack(torch.from_numpy(X).cuda()).cpu().numpy(), 3, F)
    isnan = np.isnan(X)
    assert np.isnan(got.view(np.float32)[isnan]).all()
    # sign and top bits kept, quiet bit set
    assert np.array_equal(got[isnan], (nans & 0xFFFFE000) | 0x00400000)
    assert np.array_equal(got[~isnan], (X[~isnan].view(np.uint32) + 0x1000) & 0xFFFFE000)


@pytest.mark.parametrize("unit_blocks", [0, 3])
@pytest.mark.parametrize("F", [1, 2, 64, 100, 128, 256, 257, 300, 400, 513, 602, 700])
def test_bcsr_spmm_packed(gpu, oracle, unit_blocks, F):
    """The gather over packed rows gives the oracle's TF32 product (= and +=).
    F past a whole chunk: a last chunk of at most 128 features in its own
    launch at 1 or 2 features a lane (257, 300, 513, 602); a longer one in
    the 4-feature launch, with its lanes past F idle (400, 700)."""
    from tcc_amd import swtcf

    nr, nc = 640, 900
    dst, src = skewed_coo(nr, nc, 60 + F)
    vals = np.random.default_rng(61).uniform(-1, 1, dst.size).astype(np.float32)
    X = np.random.default_rng(62).standard_normal((nc, F)).astype(np.float32)
    rowptr, colind, v = csr_of(dst, src, nr, vals)
    want = oracle.csr_spmm(rowptr, colind, v, X, use_tf32=True)
    A = swtcf.coo_to_bcsr(dev_u32(dst), dev_u32(src), torch.from_numpy(vals).cuda(), nr, nc)
    A.set_unit_blocks(unit_blocks)
    packed = swtcf.tf32_pack(torch.from_numpy(X).cuda())
    Y = swtcf.bcsr_spmm_packed(A, packed, F, torch.full((A.view.num_rowWindows * 8, F), 7.0, device="cuda"))
    assert_close(Y.cpu().numpy()[:nr], want)
    Y2 = swtcf.bcsr_spmm_packed(A, packed, F, Y.clone(), accumulate=True)
    assert_close(Y2.cpu().numpy()[:nr], 2 * want)


def test_bcsr_spmm_packed_concurrent_callers(gpu, oracle):
    """The last chunk of a packed gather runs on a second stream of the
    device, forked from and joined back into the caller's stream through
    events that all callers share under a lock.  Two host threads, each on a
    stream of its own, call it in turns (F = 602 and 300: last chunks of 90
    and 44 features, 3-block units with shared windows) into Y filled with
    NaN, and copy Y on their own stream right after each call: every copy
    holds the oracle's product, so each caller's stream waited for its own
    last chunk and the shared windows were zeroed before either launch."""
    import threading

    from tcc_amd import swtcf

    nr, nc = 640, 900
    dst, src = skewed_coo(nr, nc, 70)
    vals = np.random.default_rng(71).uniform(-1, 1, dst.size).astype(np.float32)
    rowptr, colind, v = csr_of(dst, src, nr, vals)
    A = swtcf.coo_to_bcsr(dev_u32(dst), dev_u32(src), torch.from_numpy(vals).cuda(), nr, nc)
    A.set_unit_blocks(3)
    cases = []
    for i, F in enumerate((602, 300)):
        X = np.random.default_rng(72 + i).standard_normal((nc, F)).astype(np.float32)
        cases.append((F, swtcf.tf32_pack(torch.from_numpy(X).cuda()),
                      oracle.csr_spmm(rowptr, colind, v, X, use_tf32=True)))
    torch.cuda.synchronize()
    results, errors = [[], []], []

    def caller(i):
        try:
            F, packed, _ = cases[i]
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                Y = torch.empty((A.view.num_rowWindows * 8, F), device="cuda")
                for _ in range(12):
                    Y.fill_(float("nan"))
                    swtcf.bcsr_spmm_packed(A, packed, F, Y, stream=s)
                    results[i].append(Y.clone())
            s.synchronize()
        except Exception as e:  # surfaced below
            errors.append(e)

    threads = [threading.Thread(target=caller, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for i, (F, _, want) in enumerate(cases):
        assert len(results[i]) == 12
        for Y in results[i]:
            assert_close(Y.cpu().numpy()[:nr], want)


def test_feature_table_error_is_read_and_cleared(gpu):
    """FeatureTable.error() returns TCC_DEVERR_FEATURE_INDEX after a refused
    lookup (a host row past the table, planted in id_map) and clears it: the
    next call, with no refused lookup since, returns 0."""
    from tcc_amd import gcn, swtcf

    rng = np.random.default_rng(12)
    n, F = 500, 16
    keys = np.sort(rng.choice(n * n, size=6000, replace=False))
    rows = torch.from_numpy(keys // n).cuda()
    cols = torch.from_numpy(keys % n).cuda()
    X = torch.randn(n, F, device="cuda")
    table = gcn.FeatureTable(X, cols)
    g1, _ = gcn.build_gcn_graphs(rows, cols, n, table.hot)
    g1.aggregate(F, source=table.source)
    assert table.error() == 0
    j = int(cols[~table.hot[cols]][0])  # a cold column with an edge
    table.ids[j] = n + 5  # its host row past the table: refused, read as zeros
    g1.aggregate(F, source=table.source)
    assert table.error() == swtcf.DEVERR_FEATURE_INDEX
    assert table.error() == 0
    table.ids[j] = j
    torch.cuda.synchronize()
    table.free()
