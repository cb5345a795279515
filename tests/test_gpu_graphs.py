"""HIP-graph capture of the library's launches (torch.cuda.CUDAGraph over
the kernels the C-ABI enqueues on the current stream): the BCSR gather with
its shared-window zero pass, the packed gather with its separate last chunk
(which runs on the caller's stream while it is captured, and on a second
stream of the device beside the full chunks otherwise),
the gathers over a phased BCSR (zero fill of Y, then atomics only),
the one-launch first-layer forward (fill + mixed kernel), the SWTCF SpMM,
the narrow and transposed gathers, the split-K dense products and the
hybrids (binary tiles with their slice maxima, half records and zero rows,
stored first, then the remainder's atomics; value tiles after the
remainder).  None of
them allocates, synchronises or records a memset, so each captures as is.
Each graph is replayed several times with eager work in between, new inputs
written into the captured buffers before each replay, and every replay is
compared bit for bit with an eager call on the same inputs (the same kernels
in the same order; where atomics make sums order-dependent, rel-L2 1e-6).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def dev_u32(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).cuda()


def random_coo(nd, ns, nnz, seed):
    rng = np.random.default_rng(seed)
    keys = np.sort(rng.choice(nd * ns, size=nnz, replace=False))
    return (keys // ns).astype(np.uint32), (keys % ns).astype(np.uint32)


def close(a, b, exact):
    if exact:
        return torch.equal(a, b)
    d = (a.double() - b.double()).norm() / max(b.double().norm().item(), 1e-30)
    return d.item() < 1e-6


def capture(fn):
    """Warm up on a side stream, then capture fn() into a graph."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


def replay_and_check(g, out, inputs, eager, exact, replays=3, seed=0):
    """Before each replay write fresh values into the captured inputs, do
    some unrelated eager work, replay, and compare with eager()."""
    rng = np.random.default_rng(seed)
    for i in range(replays):
        for t in inputs:
            t.copy_(torch.from_numpy(rng.standard_normal(tuple(t.shape)).astype(np.float32)).cuda())
        junk = torch.randn(1 << 16, device="cuda")
        junk.mul_(2.0).sum().item()  # eager work and a synchronisation between replays
        g.replay()
        torch.cuda.synchronize()
        got = [o.clone() for o in (out if isinstance(out, (tuple, list)) else [out])]
        want = eager()
        want = want if isinstance(want, (tuple, list)) else [want]
        torch.cuda.synchronize()
        for a, b in zip(got, want):
            assert close(a, b, exact), f"replay {i}"


def test_graph_bcsr_gathers():
    """Plain gather with 3-block units (shared windows: zero pass + atomics)
    and the packed gather at F = 300 (a last chunk of 44 features)."""
    from tcc_amd import swtcf

    nr, nc = 900, 1100
    dst, src = random_coo(nr, nc, 20000, 1)
    vals = torch.from_numpy(np.random.default_rng(2).uniform(-1, 1, dst.size).astype(np.float32)).cuda()
    A = swtcf.coo_to_bcsr(dev_u32(dst), dev_u32(src), vals, nr, nc).set_unit_blocks(3)
    X = torch.randn(nc, 128, device="cuda")
    Y = torch.empty(A.view.num_rowWindows * 8, 128, device="cuda")
    X3 = torch.randn(nc, 300, device="cuda")
    P = torch.empty(swtcf._lib.lib().tcc_tf32_packed_bytes(nc, 300) + 16, dtype=torch.uint8, device="cuda")
    Y3 = torch.empty(A.view.num_rowWindows * 8, 300, device="cuda")

    def run():
        swtcf.bcsr_spmm(A, X, Y)
        swtcf.bcsr_spmm_packed(A, swtcf.tf32_pack(X3, out=P), 300, Y3)
        return Y, Y3

    g, out = capture(run)
    replay_and_check(g, out, [X, X3], lambda: [swtcf.bcsr_spmm(A, X), swtcf.bcsr_spmm_packed(A, swtcf.tf32_pack(X3), 300)],
                     exact=False)


def test_graph_phased_gathers():
    """A 4-phase BCSR at F = 300 (a full chunk and a 44-feature last chunk):
    the Y zero fill and the all-atomic plain and packed gathers."""
    from tcc_amd import swtcf

    nr, nc, F = 700, 900, 300
    dst, src = random_coo(nr, nc, 30000, 9)
    vals = torch.from_numpy(np.random.default_rng(10).uniform(-1, 1, dst.size).astype(np.float32)).cuda()
    A = swtcf.coo_to_bcsr(dev_u32(dst), dev_u32(src), vals, nr, nc, phases=4).set_unit_blocks(5)
    X = torch.randn(nc, F, device="cuda")
    Y = torch.empty(A.out_windows * 8, F, device="cuda")
    Yp = torch.empty_like(Y)
    P = torch.empty(swtcf._lib.lib().tcc_tf32_packed_bytes(nc, F) + 16, dtype=torch.uint8, device="cuda")

    def run():
        swtcf.bcsr_spmm(A, X, Y)
        swtcf.bcsr_spmm_packed(A, swtcf.tf32_pack(X, out=P), F, Yp)
        return Y, Yp

    g, out = capture(run)
    replay_and_check(g, out, [X], lambda: [swtcf.bcsr_spmm(A, X), swtcf.bcsr_spmm_packed(A, swtcf.tf32_pack(X), F)],
                     exact=False, seed=11)


def test_graph_mixed_forward():
    from tcc_amd import swtcf
    from tcc_amd.hostmem import PinnedArray

    nr = nc = 1200
    F = 100
    dst, src = random_coo(nr, nc, 25000, 3)
    rng = np.random.default_rng(4)
    hot_ids = np.sort(rng.choice(nc, size=nc // 4, replace=False))
    csm = np.full(nc, -1, np.int32)
    csm[hot_ids] = np.arange(hot_ids.size, dtype=np.int32)
    hot = torch.empty(hot_ids.size, F, device="cuda")
    cpu = PinnedArray((nc, F))
    ptrs = torch.tensor([hot.data_ptr()], dtype=torch.int64, device="cuda")
    idm = torch.from_numpy(np.arange(nc, dtype=np.int32)).cuda()
    csm_d = torch.from_numpy(csm).cuda()
    src_desc = swtcf.feature_source(idm, csm_d, ptrs, hot_ids.size, cpu.device_ptr, nc * F)
    h = csm[src] >= 0
    A = swtcf.coo_to_bcsr(dev_u32(dst[h]), dev_u32(src[h]), None, nr, nc)
    B = swtcf.coo_to_bcsc(dev_u32(dst[~h]), dev_u32(src[~h]), None, nr, nc)
    C = torch.empty((A.view.num_rowWindows + 1) * 8, F, device="cuda")
    feats = torch.empty(nc, F, device="cuda")
    hot_idx = torch.from_numpy(hot_ids.astype(np.int64)).cuda()

    def run():
        return swtcf.spmm_cnic_forward_mixed(A, B, src_desc, C, F)

    g, out = capture(run)

    def eager():
        return swtcf.spmm_cnic_forward_mixed(A, B, src_desc, torch.empty_like(C), F)

    rng2 = np.random.default_rng(5)
    for i in range(3):
        feats.copy_(torch.from_numpy(rng2.standard_normal((nc, F)).astype(np.float32)).cuda())
        hot.copy_(feats[hot_idx])
        torch.cuda.synchronize()
        cpu.array[:] = feats.cpu().numpy()
        torch.randn(1 << 16, device="cuda").sum().item()
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        want = eager()
        torch.cuda.synchronize()
        assert close(got, want, exact=False), f"replay {i}"
    cpu.free()


def test_graph_swtcf_and_narrow_and_transpose():
    from tcc_amd import swtcf

    nr, nc = 1000, 1300
    dst, src = random_coo(nr, nc, 18000, 6)
    m = swtcf.DeviceSWTCFMatrix(nr, nc, dst.size, 16)
    ws = swtcf.SWTCFConvertWorkspace(dst.size, nc, 16)
    swtcf.convertCOOToSWTCF(dev_u32(dst), dev_u32(src), dst.size, m, ws)
    A = swtcf.coo_to_bcsr(dev_u32(dst), dev_u32(src), None, nr, nc)
    B = swtcf.coo_to_bcsc(dev_u32(dst), dev_u32(src), None, nr, nc)
    X = torch.randn(nc, 128, device="cuda")
    Ys = torch.empty(nr, 128, device="cuda")
    X2 = torch.randn(nc, 2, device="cuda")
    Y2 = torch.empty(A.view.num_rowWindows * 8, 2, device="cuda")
    dY = torch.randn(nr, 64, device="cuda")
    dX = torch.empty(B.view.num_colWindows * 8, 64, device="cuda")

    def run():
        Ys.zero_()  # a fill kernel, not a memset node
        swtcf.swtcf_spmm(m, X, Ys, 12)
        swtcf.bcsr_spmm(A, X2, Y2)
        swtcf.bcsc_transpose_spmm(B, dY, dX)
        return Ys, Y2, dX

    g, out = capture(run)

    def eager():
        Ye = torch.zeros(nr, 128, device="cuda")
        swtcf.swtcf_spmm(m, X, Ye, 12)
        return Ye, swtcf.bcsr_spmm(A, X2), swtcf.bcsc_transpose_spmm(B, dY)

    replay_and_check(g, out, [X, X2, dY], eager, exact=False, seed=7)


def test_graph_dense_products():
    from tcc_amd import swtcf

    K, M, N = 20000, 100, 256
    Am = torch.randn(K, M, device="cuda")
    Bm = torch.randn(K, N, device="cuda")
    AX = torch.randn(K, 100, device="cuda")
    H = torch.relu(torch.randn(K, 256, device="cuda"))
    G = torch.randn(K, 2, device="cuda")
    W2 = torch.randn(256, 2, device="cuda")

    def run():
        C = swtcf.dense_tn(Am, Bm)
        dW1, dW2 = swtcf.gcn_relu_grad(AX, H, G, W2)
        return C, dW1, dW2

    g, out = capture(run)
    # fixed-order split-K sums: replays equal the eager call bit for bit
    replay_and_check(g, out, [Am, Bm, AX, G], lambda: [swtcf.dense_tn(Am, Bm), *swtcf.gcn_relu_grad(AX, H, G, W2)],
                     exact=True, seed=8)


def test_graph_hybrids():
    """The binary hybrid at F = 300 (the remainder's pack with the slice
    maxima, the slice scales, half records, the tiles stored first with the
    rows they do not cover zeroed, then the 4-phase remainder's atomics) and
    the split value-tile hybrid (the remainder first, then the tiles added),
    each with its workspace allocated before capture."""
    from tcc_amd import swtcf

    nr, nc, F = 700, 900, 300
    dst, src = random_coo(nr, nc, 30000, 21)
    rng = np.random.default_rng(22)
    rs = torch.from_numpy(rng.uniform(0.1, 1.0, nr).astype(np.float32)).cuda()
    cs = torch.from_numpy(rng.uniform(0.1, 1.0, nc).astype(np.float32)).cuda()
    vals = torch.from_numpy(rng.uniform(-1, 1, dst.size).astype(np.float32)).cuda()
    Hb = swtcf.coo_to_hybrid_scaled(dev_u32(dst), dev_u32(src), nr, nc, rs, cs, min_step_nnz=190, group_blocks=16,
                                    phases=4)
    Hv = swtcf.coo_to_hybrid(dev_u32(dst), dev_u32(src), vals, nr, nc, min_tile_nnz=12, group_blocks=8,
                             tile_format=swtcf.TILES_BF16X2, phases=4)
    for H in (Hb, Hv):
        assert H.view.tiles.num_steps > 0 and H.rest.view.num_TCBlocks > 0
    X = torch.randn(nc, F, device="cuda")
    wb = torch.empty(Hb.workspace_bytes(F) + 16, dtype=torch.uint8, device="cuda")
    wv = torch.empty(Hv.workspace_bytes(F) + 16, dtype=torch.uint8, device="cuda")
    Yb = torch.empty(Hb.out_rows, F, device="cuda")
    Yv = torch.empty(Hv.out_rows, F, device="cuda")

    def run():
        swtcf.hybrid_spmm(Hb, X, Yb, workspace=wb)
        swtcf.hybrid_spmm(Hv, X, Yv, workspace=wv)
        return Yb, Yv

    g, out = capture(run)
    replay_and_check(g, out, [X], lambda: [swtcf.hybrid_spmm(Hb, X), swtcf.hybrid_spmm(Hv, X)], exact=False,
                     seed=23)
