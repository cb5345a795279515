"""The `spmm_cnic` extension: import/exports on CPU, and on the GPU every call
form of the reference (spmm_cnic/src/bindings/module.cu:344-365 and
train/tcgnn_conv_release.py:116-130, 324) against the oracle."""
import ctypes
import os
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXPORTS = ["forward_tensorcore_mixed", "forward_tensorcore", "read_cpu_feature_cache", "read_gpu0_feature_cache",
           "initialize", "space_malloc", "finalize", "freeMatC", "set_graph_plans", "release_plans", "graph_plans"]


def import_ext():
    sys.path.insert(0, os.path.join(ROOT, "tcc_amd"))
    try:
        import spmm_cnic  # the name the training scripts import
    finally:
        sys.path.pop(0)
    return spmm_cnic


def test_extension_imports_and_exports():
    m = import_ext()
    for name in EXPORTS:
        assert hasattr(m, name), name
    # both call forms are overloads of the same names
    assert "Overloaded function" in m.forward_tensorcore.__doc__
    assert "Overloaded function" in m.forward_tensorcore_mixed.__doc__


def _blocks(dst, src, nr, nc, vals=None):
    import oracle

    r64 = dst.astype(np.int64)
    order = np.lexsort((src, dst))
    rowptr = np.zeros(nr + 1, np.int64)
    rowptr[1:] = np.cumsum(np.bincount(dst, minlength=nr))
    bcsr = oracle.bcsr_build(nr, nc, rowptr, src[order], None if vals is None else vals[order])
    order = np.lexsort((r64, src))
    colptr = np.zeros(nc + 1, np.int64)
    colptr[1:] = np.cumsum(np.bincount(src, minlength=nc))
    bcsc = oracle.bcsc_build(nr, nc, colptr, dst[order], None if vals is None else vals[order])
    return bcsr, bcsc


def _dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    if a.dtype == np.uint64:
        a = a.view(np.int64)
    return torch.from_numpy(a).cuda()


def _args(bcsr, bcsc, with_data):
    r = [bcsr["num_rows"], bcsr["num_cols"], bcsr["nnz"], bcsr["num_TCBlocks"], bcsr["num_rowWindows"],
         _dev(bcsr["rowWindowOffset"]), _dev(bcsr["tcOffset"]), _dev(bcsr["sparseA2B"]), _dev(bcsr["tcLocalBit"])]
    if with_data:
        r.append(_dev(bcsr["data"]))
    c = [bcsc["num_rows"], bcsc["num_cols"], bcsc["nnz"], bcsc["num_TCBlocks"], bcsc["num_colWindows"],
         _dev(bcsc["colWindowOffset"]), _dev(bcsc["tcOffset"]), _dev(bcsc["sparseA2C"]), _dev(bcsc["tcLocalBit"])]
    if with_data:
        c.append(_dev(bcsc["data"]))
    return r + c


def _split(nr, nc, nnz, seed):
    rng = np.random.default_rng(seed)
    keys = np.sort(rng.choice(nr * nc, size=nnz, replace=False))
    dst, src = (keys // nc).astype(np.uint32), (keys % nc).astype(np.uint32)
    hot = rng.random(nc) < 0.25
    return dst, src, hot


def _want(dst, src, nr, X):
    import oracle

    order = np.lexsort((src, dst))
    rowptr = np.zeros(nr + 1, np.int64)
    rowptr[1:] = np.cumsum(np.bincount(dst, minlength=nr))
    return oracle.csr_spmm(rowptr, src[order], None, X, use_tf32=True)


def _rel(a, b):
    return np.linalg.norm(a - b) / np.linalg.norm(b)


@pytest.mark.gpu
def test_forward_tensorcore_both_forms(gpu):
    m = import_ext()
    nr = nc = 700
    F = 64
    dst, src, hot = _split(nr, nc, 9000, 1)
    h = hot[src]
    bcsr, _ = _blocks(dst[h], src[h], nr, nc)
    _, bcsc = _blocks(dst[~h], src[~h], nr, nc)
    X = np.random.default_rng(2).standard_normal((nc, F)).astype(np.float32)
    x = torch.from_numpy(X).cuda().flatten().contiguous()
    want = _want(dst, src, nr, X)
    # Python-caller form (train/tcgnn_conv_release.py:124-130)
    out = m.forward_tensorcore(*_args(bcsr, bcsc, True), F, x)
    assert out.shape == (nr * F,)
    assert _rel(out.reshape(nr, F).cpu().numpy(), want) < 1e-5
    m.freeMatC()
    # compiled form with device_id and a space_malloc buffer (module.cu:192-273)
    m.initialize(0)
    caps = m.space_malloc(0, (bcsr["num_rowWindows"] + 1) * 8 * F)
    out2 = m.forward_tensorcore(*_args(bcsr, bcsc, False), F, x, 0, caps[0])
    assert _rel(out2.reshape(nr, F).cpu().numpy(), want) < 1e-5
    torch.cuda.synchronize()
    m.finalize(0)


@pytest.mark.gpu
def test_forward_tensorcore_mixed_forms(gpu):
    from tcc_amd.hostmem import PinnedArray

    m = import_ext()
    nr = nc = 800
    F = 100
    dst, src, _ = _split(nr, nc, 10000, 3)
    rng = np.random.default_rng(4)
    feats = rng.standard_normal((nc, F)).astype(np.float32)
    hot_ids = np.sort(rng.choice(nc, size=nc // 5, replace=False))
    csm = np.full(nc, -1, np.int32)
    csm[hot_ids] = np.arange(hot_ids.size, dtype=np.int32)
    ids = np.arange(nc, dtype=np.int32)
    hot_mask = csm[src] >= 0
    bcsr, _ = _blocks(dst[hot_mask], src[hot_mask], nr, nc)
    _, bcsc = _blocks(dst[~hot_mask], src[~hot_mask], nr, nc)
    cache = torch.from_numpy(feats[hot_ids]).cuda()
    ptr_table = torch.tensor([cache.data_ptr()], dtype=torch.int64, device="cuda")
    cpu = PinnedArray((nc, F))
    cpu.array[:] = feats
    PyCapsule_New = ctypes.pythonapi.PyCapsule_New
    PyCapsule_New.restype = ctypes.py_object
    PyCapsule_New.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p]
    cpu_cap = PyCapsule_New(cpu._ptr.value, None, None)
    gpu_cap = PyCapsule_New(ptr_table.data_ptr(), None, None)
    want = _want(dst, src, nr, feats)
    ids_d = torch.from_numpy(ids).cuda()
    csm_d = torch.from_numpy(csm).cuda()
    # Python-caller form (train/tcgnn_conv_release.py:116-122): 27 arguments
    out = m.forward_tensorcore_mixed(*_args(bcsr, bcsc, True), nc * F, hot_ids.size, F,
                                     ids_d, cpu_cap, csm_d, gpu_cap)
    assert _rel(out.reshape(nr, F).cpu().numpy(), want) < 1e-5
    m.freeMatC()
    # compiled form with x (module.cu:100-190): computes with x
    caps = m.space_malloc(0, (bcsr["num_rowWindows"] + 1) * 8 * F)
    x = torch.from_numpy(feats).cuda().flatten()
    out2 = m.forward_tensorcore_mixed(*_args(bcsr, bcsc, False), nc * F, hot_ids.size, F,
                                      ids_d, cpu_cap, csm_d, gpu_cap,
                                      x, 0, caps[0])
    assert _rel(out2.reshape(nr, F).cpu().numpy(), want) < 1e-5
    # mixed-memory compiled form (module.cu:21-97): reads the feature source
    out3 = m.forward_tensorcore_mixed(*_args(bcsr, bcsc, False), nc * F, hot_ids.size, F,
                                      ids_d, cpu_cap, csm_d, gpu_cap,
                                      0, caps[1])
    assert _rel(out3.reshape(nr, F).cpu().numpy(), want) < 1e-5
    # valid maps: no lookup was refused
    assert m.feature_error(0) == 0
    torch.cuda.synchronize()
    m.finalize(0)
    cpu.free()


def _hub_coo(nr, nc, nnz, seed):
    from test_gpu_hybrid import random_coo

    return random_coo(nr, nc, nnz, seed, True)


@pytest.mark.gpu
@pytest.mark.parametrize("F", [100, 602])
def test_forward_tensorcore_packs_x_for_high_reuse(gpu, F):
    """Rows gathered >= 16 times on average: the extension packs x into exact
    TF32 rows first (tcc_spmm_cnic_forward_ws); the product is the same."""
    from tcc_amd import _lib, swtcf

    m = import_ext()
    nr, nc = 2000, 300
    dst, src, hot = _split(nr, nc, 60000, 5)
    h = hot[src]
    bcsr, _ = _blocks(dst[h], src[h], nr, nc)
    _, bcsc = _blocks(dst[~h], src[~h], nr, nc)
    A = swtcf.host_to_bcsr(bcsr)
    need = _lib.lib().tcc_spmm_cnic_forward_workspace_bytes(ctypes.byref(A.view), F)
    assert need == _lib.lib().tcc_tf32_packed_bytes(nc, F) + 16  # packing pays here
    X = np.random.default_rng(6).standard_normal((nc, F)).astype(np.float32)
    out = m.forward_tensorcore(*_args(bcsr, bcsc, True), F, torch.from_numpy(X).cuda().flatten())
    assert _rel(out.reshape(nr, F).cpu().numpy(), _want(dst, src, nr, X)) < 1e-5
    m.freeMatC()


@pytest.mark.gpu
def test_hybrid_from_bcsr_matches_the_coo_build(gpu, oracle):
    """tcc_hybrid_from_bcsr of the oracle's BCSR holds exactly the arrays of
    the binary hybrid built from the same COO; with values, the split-TF32
    hybrid's product equals the oracle's."""
    from test_gpu_hybrid import dev_u32
    from tcc_amd import swtcf

    nr, nc, F = 700, 900, 96
    dst, src = _hub_coo(nr, nc, 60000, 31)
    vals = np.random.default_rng(32).uniform(-1, 1, dst.size).astype(np.float32)
    bcsr, _ = _blocks(dst, src, nr, nc, vals)
    A = swtcf.host_to_bcsr(bcsr, use_data=True)
    Hb = swtcf.hybrid_from_bcsr(A, min_step_nnz=16)
    Hc = swtcf.coo_to_hybrid_scaled(dev_u32(dst), dev_u32(src), nr, nc, min_step_nnz=16, phases=1)
    hb, hc = Hb.to_host(), Hc.to_host()
    for k in ("rowOrder", "hubColOrder", "groupStepOffset", "stepCol", "units", "unitOrder", "unitPartial",
              "sharedGroups", "tileMasks"):
        assert np.array_equal(hb[k], hc[k]), k
    for k in ("rowWindowOffset", "sparseA2B", "tcLocalBit"):
        assert np.array_equal(hb["rest"][k], hc["rest"][k]), k
    X = np.random.default_rng(33).standard_normal((nc, F)).astype(np.float32)
    Xd = torch.from_numpy(X).cuda()
    assert _rel(swtcf.hybrid_spmm(Hb, Xd).cpu().numpy()[:nr], _want(dst, src, nr, X)) < 1e-5
    Hv = swtcf.hybrid_from_bcsr(A, use_values=True)
    order = np.lexsort((src, dst))
    rowptr = np.zeros(nr + 1, np.int64)
    rowptr[1:] = np.cumsum(np.bincount(dst, minlength=nr))
    want_v = oracle.csr_spmm(rowptr, src[order], vals[order], X, use_tf32=True)
    assert _rel(swtcf.hybrid_spmm(Hv, Xd).cpu().numpy()[:nr], want_v) < 1e-5


@pytest.mark.gpu
def test_forward_tensorcore_graph_plans(gpu, oracle):
    """set_graph_plans(n): the extension keeps a per-graph plan (dense tiles
    on MFMA + gather) from the first call on any graph, finds it again by a
    hash of the BCSR arrays, keeps at most n, and drops them on
    release_plans(); with set_use_values the plan holds the values.  Every
    product against the oracle."""
    m = import_ext()
    nr, nc, F = 600, 700, 130
    graphs = []
    for seed in (41, 42, 43):
        dst, src = _hub_coo(nr, nc, 50000, seed)
        bcsr, bcsc = _blocks(dst, src, nr, nc)
        empty = _blocks(np.zeros(0, np.uint32), np.zeros(0, np.uint32), nr, nc)[1]
        graphs.append((dst, src, _args(bcsr, empty, True)))
    X = np.random.default_rng(44).standard_normal((nc, F)).astype(np.float32)
    x = torch.from_numpy(X).cuda().flatten()
    try:
        m.set_graph_plans(2)
        for _ in range(2):  # the second call finds the plan
            dst, src, args = graphs[0]
            out = m.forward_tensorcore(*args, F, x)
            assert _rel(out.reshape(nr, F).cpu().numpy(), _want(dst, src, nr, X)) < 1e-5
            assert m.graph_plans() == 1
        for dst, src, args in graphs[1:]:
            out = m.forward_tensorcore(*args, F, x)
            assert _rel(out.reshape(nr, F).cpu().numpy(), _want(dst, src, nr, X)) < 1e-5
        assert m.graph_plans() == 2  # the least recently used one was released
        # the compiled form with its caller-owned denseC
        dst, src, args = graphs[2]
        args_nodata = args[:9] + args[10:19]
        caps = m.space_malloc(0, (int(args[4]) + 1) * 8 * F)
        out = m.forward_tensorcore(*args_nodata, F, x, 0, caps[0])
        assert _rel(out.reshape(nr, F).cpu().numpy(), _want(dst, src, nr, X)) < 1e-5
        # values: a plan of its own, over the data tensors
        dst, src, _ = graphs[0]
        vals = np.random.default_rng(45).uniform(-1, 1, dst.size).astype(np.float32)
        bcsr, _ = _blocks(dst, src, nr, nc, vals)
        empty = _blocks(np.zeros(0, np.uint32), np.zeros(0, np.uint32), nr, nc)[1]
        m.set_use_values(True)
        out = m.forward_tensorcore(*_args(bcsr, empty, True), F, x)
        order = np.lexsort((src, dst))
        rowptr = np.zeros(nr + 1, np.int64)
        rowptr[1:] = np.cumsum(np.bincount(dst, minlength=nr))
        want_v = oracle.csr_spmm(rowptr, src[order], vals[order], X, use_tf32=True)
        assert _rel(out.reshape(nr, F).cpu().numpy(), want_v) < 1e-5
        m.release_plans()
        assert m.graph_plans() == 0
    finally:
        m.set_use_values(False)
        m.set_graph_plans(-1)  # the automatic default
        m.freeMatC()
        torch.cuda.synchronize()
        m.finalize(0)


@pytest.mark.gpu
def test_forward_tensorcore_automatic_plans(gpu, oracle):
    """An unchanged caller: by default a large graph with long row windows
    (>= 65,536 blocks, >= 64 a window) gets a plan from the second call
    that finds the same arrays (a device hash of rowWindowOffset, sparseA2B
    and tcLocalBit); the first call runs the packed gather.  A bitmap
    rewritten in place hashes differently: that call runs the default path
    on the new graph, and the next call builds the new graph's plan in
    place of the old one; restored, the first graph's plan is built again.
    Every product against the oracle."""
    m = import_ext()
    nr, nc, F = 512, 60000, 96
    rng = np.random.default_rng(51)
    keys = np.unique(rng.integers(0, nr * nc, size=1_300_000, dtype=np.int64))
    dst, src = (keys // nc).astype(np.uint32), (keys % nc).astype(np.uint32)
    bcsr, _ = _blocks(dst, src, nr, nc)
    assert bcsr["num_TCBlocks"] >= 65536 and bcsr["num_TCBlocks"] >= 64 * bcsr["num_rowWindows"]
    empty = _blocks(np.zeros(0, np.uint32), np.zeros(0, np.uint32), nr, nc)[1]
    args = _args(bcsr, empty, True)
    X = np.random.default_rng(52).standard_normal((nc, F)).astype(np.float32)
    x = torch.from_numpy(X).cuda().flatten()
    try:
        m.set_graph_plans(-1)
        m.release_plans()
        want = _want(dst, src, nr, X)
        for call, plans in ((1, 0), (2, 1), (3, 1)):
            out = m.forward_tensorcore(*args, F, x)
            assert _rel(out.reshape(nr, F).cpu().numpy(), want) < 1e-5, call
            assert m.graph_plans() == plans, call
            m.freeMatC()
        # one entry of block 0 removed in place
        b0 = int(np.uint64(bcsr["tcLocalBit"][0]))
        i = (b0 & -b0).bit_length() - 1
        w0 = int(np.searchsorted(bcsr["rowWindowOffset"], 0, side="right")) - 1
        row, col = 8 * w0 + i // 8, int(bcsr["sparseA2B"][i % 8])
        args[8][0] = int(np.array([b0 & ~(1 << i)], np.uint64).view(np.int64)[0])
        keep = ~((dst == row) & (src == col))
        assert keep.sum() == dst.size - 1
        want2 = _want(dst[keep], src[keep], nr, X)
        for call, plans in ((4, 1), (5, 1)):
            out = m.forward_tensorcore(*args, F, x)
            assert _rel(out.reshape(nr, F).cpu().numpy(), want2) < 1e-5, call
            assert m.graph_plans() == plans, call
            m.freeMatC()
        # the entry restored: the first graph again, whose plan the second's
        # replaced; its plan is built again and the second's released
        args[8][0] = int(np.array([b0], np.uint64).view(np.int64)[0])
        for call in (6, 7):
            out = m.forward_tensorcore(*args, F, x)
            assert _rel(out.reshape(nr, F).cpu().numpy(), want) < 1e-5, call
            assert m.graph_plans() == 1, call
            m.freeMatC()
        # turned off: the default path, no plan kept
        m.set_graph_plans(0)
        assert m.graph_plans() == 0
        out = m.forward_tensorcore(*args, F, x)
        assert _rel(out.reshape(nr, F).cpu().numpy(), want) < 1e-5
    finally:
        m.set_graph_plans(-1)
        m.freeMatC()
        torch.cuda.synchronize()
