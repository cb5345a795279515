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
  cut at Y's end: sentinel rows right after Y stay untouched.
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
