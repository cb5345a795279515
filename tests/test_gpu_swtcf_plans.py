"""Plans for repeated SWTCF SpMMs (tcc_swtcf_set_plans; launchSWTCFSpMM's
product, src/swtcf_spmm.cu:437-466, through the binary hybrid of the same
pattern).

Checked through the C-ABI, on an R-MAT matrix above the plan gate (4M edges
of capacity, 64 entries per row on average):
- the first call on a matrix runs the SWTCF kernel; the second builds the
  plan and runs it; the third reuses it (tcc_swtcf_plans_built counts);
- the planned products against the fp64 CSR oracle over TF32(X) at rel-L2
  <= 1e-5 (every entry multiplies TF32(X) exactly, sums in fp32), and
  against the kernel's product (TF32 only for tiles of >= tcThreshold
  entries) at the north star's 1e-3; Y += AX adds into what Y holds;
- a matrix converted again in place from another COO hashes differently:
  its first call is the kernel's again, and correct;
- tcThreshold 65 (the reference's pure fp32 path) and tcc_swtcf_set_plans(0)
  never plan;
- another feature width (tcc_swtcf_spmm_f, F = 72) reuses the plan with a
  workspace of its own size;
- launchSWTCFSpMMQuantized plans too, dequantizing X into the plan's buffer;
- matrices below the hybrid's gate (at least 2^18 edges) plan the BCSR
  gather of their pattern, over X or (rows gathered 16 times or more) over
  X packed to TF32 rows; with rows not a multiple of 8 the last window is
  cut at Y's end: sentinel rows right after Y stay untouched;
- two matrices in turn: with one plan kept, each build releases the other
  matrix's plan and its next call builds it again; with two, both stay.
"""
import numpy as np
import pytest
import torch

from test_gpu_hybrid import oracle_product, rel_l2

pytestmark = pytest.mark.gpu


def rmat_coo(n, nnz, seed):
    from tcc_amd.graphs import rmat_graph

    rows, cols = rmat_graph(n, nnz, seed, device="cuda")
    return rows.to(torch.int32).contiguous(), cols.to(torch.int32).contiguous()


def convert(swtcf, m, ws, r32, c32):
    swtcf.convertCOOToSWTCF(r32, c32, r32.numel(), m, ws)
    assert ws.device_error() == 0


@pytest.fixture
def plans():
    from tcc_amd import _lib

    L = _lib.lib()
    L.tcc_swtcf_release_plans()
    L.tcc_swtcf_set_plans(1)
    yield L
    L.tcc_swtcf_release_plans()
    L.tcc_swtcf_set_plans(1)


def test_plan_built_on_second_call(gpu, oracle, plans):
    from tcc_amd import swtcf

    n, E, F = 40000, 4_400_000, 128
    r32, c32 = rmat_coo(n, E, 11)
    m = swtcf.DeviceSWTCFMatrix(n, n, E, 16)
    ws = swtcf.SWTCFConvertWorkspace(E, n, 16)
    convert(swtcf, m, ws, r32, c32)
    dst, src = r32.cpu().numpy().view(np.uint32), c32.cpu().numpy().view(np.uint32)
    X = np.random.default_rng(2).standard_normal((n, F)).astype(np.float32)
    Xd = torch.from_numpy(X).cuda()
    want = oracle_product(oracle, dst, src, None, n, X)  # fp64 over TF32(X)
    b0 = plans.tcc_swtcf_plans_built()
    Y1 = torch.zeros((n, F), device="cuda")
    swtcf.launchSWTCFSpMM(m, Xd, Y1)
    torch.cuda.synchronize()
    assert plans.tcc_swtcf_plans_built() == b0, "the first call must run the SWTCF kernel"
    Y2 = torch.zeros((n, F), device="cuda")
    swtcf.launchSWTCFSpMM(m, Xd, Y2)
    torch.cuda.synchronize()
    assert plans.tcc_swtcf_plans_built() == b0 + 1, "the second call must build the plan"
    Y0 = np.random.default_rng(3).standard_normal((n, F)).astype(np.float32)
    Y3 = torch.from_numpy(Y0).cuda()
    swtcf.launchSWTCFSpMM(m, Xd, Y3)  # Y += AX through the kept plan
    torch.cuda.synchronize()
    assert plans.tcc_swtcf_plans_built() == b0 + 1
    y1, y2, y3 = Y1.cpu().numpy(), Y2.cpu().numpy(), Y3.cpu().numpy()
    e2, e3 = rel_l2(y2, want), rel_l2(y3 - Y0, want)
    e1 = rel_l2(y1, y2)
    print(f"plans: kernel vs plan {e1:.2e}, plan vs TF32 oracle {e2:.2e}, accumulate {e3:.2e}", flush=True)
    assert e2 <= 1e-5 and e3 <= 1e-5 and e1 <= 1e-3
    # another feature width through tcc_swtcf_spmm_f: the same plan, a workspace of its size
    F2 = 72
    X2 = np.ascontiguousarray(X[:, :F2])
    Y4 = torch.zeros((n, F2), device="cuda")
    swtcf.swtcf_spmm(m, torch.from_numpy(X2).cuda(), Y4)
    torch.cuda.synchronize()
    assert plans.tcc_swtcf_plans_built() == b0 + 1
    assert rel_l2(Y4.cpu().numpy(), want[:, :F2]) <= 1e-5
    # the pure fp32 path (tcThreshold > 64) never plans
    Y5 = torch.zeros((n, F), device="cuda")
    swtcf.launchSWTCFSpMM(m, Xd, Y5, 65)
    torch.cuda.synchronize()
    assert rel_l2(Y5.cpu().numpy(), y1) <= 1e-3 and rel_l2(Y5.cpu().numpy(), want) <= 1e-3
    # the same arrays converted from another COO: a new hash, the kernel's product first
    r32b, c32b = rmat_coo(n, E, 12)
    convert(swtcf, m, ws, r32b, c32b)
    dstb, srcb = r32b.cpu().numpy().view(np.uint32), c32b.cpu().numpy().view(np.uint32)
    Y6 = torch.zeros((n, F), device="cuda")
    swtcf.launchSWTCFSpMM(m, Xd, Y6)
    torch.cuda.synchronize()
    assert plans.tcc_swtcf_plans_built() == b0 + 1
    assert rel_l2(Y6.cpu().numpy(), oracle_product(oracle, dstb, srcb, None, n, X)) <= 1e-3
    m.free()
    ws.free()


def test_plans_off(gpu, oracle, plans):
    from tcc_amd import swtcf

    plans.tcc_swtcf_set_plans(0)
    n, E, F = 30000, 4_300_000, 64
    r32, c32 = rmat_coo(n, E, 13)
    m = swtcf.DeviceSWTCFMatrix(n, n, E, 16)
    ws = swtcf.SWTCFConvertWorkspace(E, n, 16)
    convert(swtcf, m, ws, r32, c32)
    X = torch.randn((n, F), device="cuda")
    b0 = plans.tcc_swtcf_plans_built()
    for _ in range(3):
        Y = torch.zeros((n, F), device="cuda")
        swtcf.swtcf_spmm(m, X, Y)
    torch.cuda.synchronize()
    assert plans.tcc_swtcf_plans_built() == b0
    dst, src = r32.cpu().numpy().view(np.uint32), c32.cpu().numpy().view(np.uint32)
    assert rel_l2(Y.cpu().numpy(), oracle_product(oracle, dst, src, None, n, X.cpu().numpy())) <= 1e-3
    m.free()
    ws.free()


@pytest.mark.parametrize("n,E,F", [(40003, 420_000, 128), (40005, 1_300_000, 72), (40001, 500_000, 13)])
def test_gather_plan(gpu, oracle, plans, n, E, F):
    """Below the hybrid's gate the plan is the BCSR gather of the pattern:
    over X at 10 entries a row (F = 128; F = 13, which the wide gather takes
    because of the row limit), over packed TF32 rows at 32 (F = 72).  Each
    call adds into Y = buf[:n], where buf holds 8 sentinel rows after Y."""
    from tcc_amd import swtcf

    r32, c32 = rmat_coo(n, E, 21)
    m = swtcf.DeviceSWTCFMatrix(n, n, E, 16)
    ws = swtcf.SWTCFConvertWorkspace(E, n, 16)
    convert(swtcf, m, ws, r32, c32)
    # the case takes the path it is meant for: packed rows where the BCSR
    # gathers each row 16 times or more on average
    A = swtcf.coo_to_bcsr(r32, c32, None, n, n)
    assert (8 * A.view.num_TCBlocks >= 16 * n) == (F == 72), A.view.num_TCBlocks
    A.release()
    dst, src = r32.cpu().numpy().view(np.uint32), c32.cpu().numpy().view(np.uint32)
    X = np.random.default_rng(22).standard_normal((n, F)).astype(np.float32)
    Xd = torch.from_numpy(X).cuda()
    want = oracle_product(oracle, dst, src, None, n, X)
    Y0 = np.random.default_rng(23).standard_normal((n, F)).astype(np.float32)
    b0 = plans.tcc_swtcf_plans_built()
    got = []
    for call in range(3):
        buf = torch.full((n + 8, F), 12345.0, device="cuda")
        buf[:n] = torch.from_numpy(Y0).cuda()
        swtcf.swtcf_spmm(m, Xd, buf[:n])
        torch.cuda.synchronize()
        assert plans.tcc_swtcf_plans_built() == b0 + (0 if call == 0 else 1), call
        b = buf.cpu().numpy()
        assert (b[n:] == 12345.0).all(), f"call {call} wrote past Y"
        got.append(b[:n] - Y0)
    e = [rel_l2(g, want) for g in got]
    print(f"gather plan n={n} E={E} F={F}: kernel {e[0]:.2e}, plan {e[1]:.2e} {e[2]:.2e}", flush=True)
    assert e[0] <= 1e-3 and e[1] <= 1e-5 and e[2] <= 1e-5
    m.free()
    ws.free()


@pytest.mark.parametrize("n,E", [(36000, 4_250_000), (30001, 500_000)])
def test_quantized_plan(gpu, oracle, plans, n, E):
    """launchSWTCFSpMMQuantized (X[src] = q[srcGlobal[src]] * scales[srcGlobal[src]],
    src/swtcf_spmm.cu:317-323) through the same plans: the first call runs
    the SWTCF kernel, the second builds the plan, which dequantizes X into
    its own buffer and runs the hybrid (or, below its gate, the gather);
    against the fp64 oracle over TF32(dequantized X) at 1e-5 (plan) and
    1e-3 (kernel)."""
    from tcc_amd import swtcf

    F = 128
    r32, c32 = rmat_coo(n, E, 14)
    m = swtcf.DeviceSWTCFMatrix(n, n, E, 16)
    ws = swtcf.SWTCFConvertWorkspace(E, n, 16)
    convert(swtcf, m, ws, r32, c32)
    rng = np.random.default_rng(15)
    N = n + 100
    q = rng.integers(-127, 128, size=(N, F), dtype=np.int8)
    scales = rng.uniform(0.001, 0.05, N).astype(np.float32)
    src_global = rng.permutation(N)[:n].astype(np.uint32)
    Xdq = (q[src_global].astype(np.float32) * scales[src_global][:, None]).astype(np.float32)
    dst, src = r32.cpu().numpy().view(np.uint32), c32.cpu().numpy().view(np.uint32)
    want = oracle_product(oracle, dst, src, None, n, Xdq)
    qd = torch.from_numpy(q).cuda()
    sd = torch.from_numpy(scales).cuda()
    gd = torch.from_numpy(src_global.view(np.int32)).cuda()
    b0 = plans.tcc_swtcf_plans_built()
    got = []
    for call in range(3):
        Y = torch.zeros((n, F), device="cuda")
        swtcf.launchSWTCFSpMMQuantized(m, qd, sd, gd, Y)
        torch.cuda.synchronize()
        assert plans.tcc_swtcf_plans_built() == b0 + (0 if call == 0 else 1), call
        got.append(Y.cpu().numpy())
    e = [rel_l2(g, want) for g in got]
    print(f"quantized: kernel {e[0]:.2e}, plan {e[1]:.2e} {e[2]:.2e}", flush=True)
    assert e[0] <= 1e-3 and e[1] <= 1e-5 and e[2] <= 1e-5
    m.free()
    ws.free()


def _fmix32(h):
    h = h ^ (h >> np.uint32(16))
    h = h * np.uint32(0x85EBCA6B)
    h = h ^ (h >> np.uint32(13))
    h = h * np.uint32(0xC2B2AE35)
    return h ^ (h >> np.uint32(16))


def hash_sums(arrays):
    """The two sums tcc_hash_arrays forms, restated in numpy: word j of
    array k (salt k + 1) with index key k32 = j ^ (j >> 32) * 0x27D4EB2F
    gives a = fmix32(w + k32 * 0x9E3779B9 + salt) into the first sum and
    fmix32(a ^ (k32 + 0x5BD1E995 * salt)) into the second (MurmurHash3's
    32-bit finalizer; 32-bit wrap-around, sums modulo 2^64)."""
    s0 = s1 = 0
    with np.errstate(over="ignore"):
        for k, w in enumerate(arrays):
            salt = np.uint32(k + 1)
            j = np.arange(w.size, dtype=np.uint64)
            k32 = (j & np.uint64(0xFFFFFFFF)).astype(np.uint32) ^ ((j >> np.uint64(32)).astype(np.uint32) * np.uint32(0x27D4EB2F))
            a = _fmix32(w + k32 * np.uint32(0x9E3779B9) + salt)
            b = _fmix32(a ^ (k32 + np.uint32(0x5BD1E995) * salt))
            s0 += int(a.astype(np.uint64).sum())
            s1 += int(b.astype(np.uint64).sum())
    return s0 % 2**64, s1 % 2**64


def test_hash_arrays_slots(gpu, plans):
    """tcc_hash_arrays writes TCC_HASH_WORDS / 2 pairs of partial sums, whose
    even and odd words add up (modulo 2^64) to the two sums of its mixing,
    restated above: checked on three arrays, one not 16-byte aligned (one
    word a thread) and one empty; changing one word changes both sums."""
    import ctypes

    rng = np.random.default_rng(31)
    host = [rng.integers(0, 2**32, size=n, dtype=np.uint64).astype(np.uint32) for n in (1_000_003, 77_777, 0)]
    dev = [torch.from_numpy(h.view(np.int32)).cuda() for h in host]
    base = torch.zeros(77_777 + 1, dtype=torch.int32, device="cuda")
    base[1:] = dev[1]
    views = [dev[0], base[1:], dev[2]]  # the second one 4 bytes past a 256-byte boundary
    out = torch.empty(64, dtype=torch.int64, device="cuda")

    def run(vs):
        ptrs = (ctypes.c_void_p * 3)(*[v.data_ptr() if v.numel() else None for v in vs])
        nbytes = (ctypes.c_uint64 * 3)(*[4 * v.numel() for v in vs])
        assert plans.tcc_hash_arrays(ptrs, nbytes, 3, ctypes.c_void_p(out.data_ptr()), None) == 0
        w = out.cpu().numpy().view(np.uint64)
        return int(w[0::2].astype(object).sum()) % 2**64, int(w[1::2].astype(object).sum()) % 2**64

    got = run(views)
    assert got == hash_sums(host)
    dev[0][500_000] ^= 1
    torch.cuda.synchronize()
    changed = run(views)
    assert changed[0] != got[0] and changed[1] != got[1]


@pytest.mark.parametrize("limit", [1, 2])
def test_two_matrices_alternate(gpu, oracle, plans, limit):
    """Two matrices multiplied in turn, each twice in a row: with one plan
    kept, building the second's plan releases the first's (the least
    recently used) but remembers the matrix, so the first's next call builds
    it again at once; with two kept, both plans stay.  Every product,
    through the kernel or a plan, against its own matrix's oracle."""
    from tcc_amd import swtcf

    plans.tcc_swtcf_set_plans(limit)
    n, E, F = 40003, 420_000, 64
    mats = []
    for seed in (31, 32):
        r32, c32 = rmat_coo(n, E, seed)
        m = swtcf.DeviceSWTCFMatrix(n, n, E, 16)
        ws = swtcf.SWTCFConvertWorkspace(E, n, 16)
        convert(swtcf, m, ws, r32, c32)
        mats.append((m, ws, r32.cpu().numpy().view(np.uint32), c32.cpu().numpy().view(np.uint32)))
    X = np.random.default_rng(33).standard_normal((n, F)).astype(np.float32)
    Xd = torch.from_numpy(X).cuda()
    want = [oracle_product(oracle, d, s, None, n, X) for _, _, d, s in mats]
    b0 = plans.tcc_swtcf_plans_built()
    order = [0, 0, 1, 1, 0, 0, 1, 1]
    # builds after each call: one plan kept rebuilds on every return, two keep both
    builds = [0, 1, 1, 2, 3, 3, 4, 4] if limit == 1 else [0, 1, 1, 2, 2, 2, 2, 2]
    for call, (k, nb) in enumerate(zip(order, builds)):
        Y = torch.zeros((n, F), device="cuda")
        swtcf.swtcf_spmm(mats[k][0], Xd, Y)
        torch.cuda.synchronize()
        assert plans.tcc_swtcf_plans_built() == b0 + nb, (limit, call)
        e = rel_l2(Y.cpu().numpy(), want[k])
        assert e <= 1e-3, (limit, call, e)
    for m, ws, _, _ in mats:
        m.free()
        ws.free()
