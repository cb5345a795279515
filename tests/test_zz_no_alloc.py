"""tcc_dense_tn_noalloc (include/tcc_gcn.h): C = A^T B with the partial
products in the library's fixed 16 MiB device array instead of a caller
workspace, called through the C-ABI.

Checked against tcc_dense_tn (the entry point it varies) on the same inputs,
on two calls in a row, the second smaller than the first (the array keeps
the first call's contents): bit for bit where both split K alike, within
fp32 summation order (rel-L2 <= 1e-6) where the 16 MiB cap takes fewer
splits (the GCN's 100 x 256 weight gradient), and both against a float64
product (rel-L2 <= 1e-5, as tests/test_gpu_dense.py).  Also accumulate,
K = 0, and the size limit."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

SCRATCH = 16 << 20


def lib():
    from tcc_amd import _lib

    return _lib.lib()


def stream():
    return torch.cuda.current_stream().cuda_stream


def with_workspace(A, B, C, accumulate):
    K, M = A.shape
    N = B.shape[1]
    L = lib()
    ws_bytes = L.tcc_dense_tn_workspace_bytes(K, M, N)
    ws = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device="cuda")
    rc = L.tcc_dense_tn(A.data_ptr(), M, B.data_ptr(), N, C.data_ptr(), N, K, M, N, int(accumulate), ws.data_ptr(),
                        ws_bytes, stream())
    assert rc == 0, L.tcc_last_error()
    return ws_bytes


def without_allocation(A, B, C, accumulate):
    K, M = A.shape
    N = B.shape[1]
    L = lib()
    rc = L.tcc_dense_tn_noalloc(A.data_ptr(), M, B.data_ptr(), N, C.data_ptr(), N, K, M, N, int(accumulate),
                                stream())
    assert rc == 0, L.tcc_last_error()


def rel_l2(a, b):
    a = a.double().cpu()
    b = b.double().cpu()
    return float((a - b).norm() / max(float(b.norm()), 1e-300))


@pytest.mark.parametrize("order", ["large_then_small", "small_then_large"])
def test_noalloc_matches_workspace_entry(gpu, order):
    shapes = [(200_000, 100, 256), (5_000, 64, 32)]  # (K, M, N): capped splits, then uncapped
    if order == "small_then_large":
        shapes = shapes[::-1] + [(3_000, 20, 2)]
    g = torch.Generator(device="cuda").manual_seed(7)
    for K, M, N in shapes:
        print(f"noalloc A^T B: K={K} M={M} N={N}", flush=True)
        A = torch.randn(K, M, device="cuda", generator=g)
        B = torch.randn(K, N, device="cuda", generator=g)
        C0 = torch.empty(M, N, device="cuda")
        C1 = torch.full((M, N), float("nan"), device="cuda")
        ws_bytes = with_workspace(A, B, C0, False)
        without_allocation(A, B, C1, False)
        torch.cuda.synchronize()
        want = A.double().t() @ B.double()
        assert rel_l2(C0, want) <= 1e-5 and rel_l2(C1, want) <= 1e-5
        if ws_bytes <= SCRATCH:
            assert torch.equal(C0, C1), "same split of K: bit for bit"
        else:
            assert rel_l2(C1, C0) <= 1e-6
        # accumulate: C += A^T B
        C2 = C1.clone()
        without_allocation(A, B, C2, True)
        torch.cuda.synchronize()
        assert rel_l2(C2, 2.0 * want) <= 1e-5


def test_noalloc_k0_and_limit(gpu):
    L = lib()
    C = torch.full((5, 7), 3.0, device="cuda")
    dummy = torch.zeros(1, device="cuda")
    assert L.tcc_dense_tn_noalloc(dummy.data_ptr(), 5, dummy.data_ptr(), 7, C.data_ptr(), 7, 0, 5, 7, 0, stream()) == 0
    torch.cuda.synchronize()
    assert torch.count_nonzero(C).item() == 0
    # M x N floats above the 16 MiB array: refused on the host, nothing launched
    rc = L.tcc_dense_tn_noalloc(dummy.data_ptr(), 2049, dummy.data_ptr(), 2049, C.data_ptr(), 2049, 16, 2049, 2049, 0,
                                stream())
    assert rc == 3
    assert b"16 MiB" in L.tcc_last_error()


def test_noalloc_under_graph_capture(gpu):
    """tcc_dense_tn_noalloc captured in a HIP graph (torch.cuda.CUDAGraph).
    Its first call on a device looks up the device array's address, so one
    uncaptured call comes first; then each of three replays, with new inputs
    written eagerly and a synchronisation between them, equals an eager
    tcc_dense_tn on the same inputs."""
    K, M, N = 20_000, 100, 64
    g = torch.Generator(device="cuda").manual_seed(11)
    A = torch.randn(K, M, device="cuda", generator=g)
    B = torch.randn(K, N, device="cuda", generator=g)
    C = torch.empty(M, N, device="cuda")
    without_allocation(A, B, C, False)  # outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        without_allocation(A, B, C, False)
    for k in range(3):
        A.copy_(torch.randn(K, M, device="cuda", generator=g))
        B.copy_(torch.randn(K, N, device="cuda", generator=g))
        ref = torch.empty(M, N, device="cuda")
        with_workspace(A, B, ref, False)
        torch.cuda.synchronize()
        C.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        print(f"noalloc graph replay {k}: rel-L2 {rel_l2(C, ref):.2e}", flush=True)
        assert rel_l2(C, ref) <= 1e-6
        assert rel_l2(C, A.double().t() @ B.double()) <= 1e-5
