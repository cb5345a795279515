"""tcc_dense_tn (C = A^T B over K rows: the GCN weight gradient
torch.mm(X_out.T, d_output), train/tcgnn_conv_release.py:150) through the
C-ABI, against float64 products of the same fp32 inputs.  Tolerance rel-L2
1e-5: fp32 MFMA products and fp32 sums over K rows split into partials; a
wrong row, column, tile or split index gives errors of order 1."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

REL = 1e-5


def rel_l2(got, want):
    got = got.double().cpu().numpy()
    want = want.double().cpu().numpy()
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


def inputs(K, M, N, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    A = torch.randn(K, M, generator=g, dtype=torch.float32)
    B = torch.randn(K, N, generator=g, dtype=torch.float32)
    return A.cuda(), B.cuda()


SHAPES = [
    (1, 1, 1), (3, 5, 7), (4, 16, 16), (17, 100, 256), (33, 2, 256), (1000, 100, 256), (4099, 256, 2),
    (777, 17, 300), (3001, 300, 40), (513, 8, 600), (100, 129, 257), (5000, 64, 64), (2047, 112, 512),
    (200003, 100, 256), (150001, 256, 2), (65537, 2, 256),
    (50000, 602, 64), (3000, 200, 17), (4099, 130, 128),  # N narrow: computed as C^T = B^T A
]


@pytest.mark.parametrize("K,M,N", SHAPES)
def test_dense_tn_matches_float64(K, M, N):
    from tcc_amd import swtcf

    A, B = inputs(K, M, N, K * 131 + M * 7 + N)
    C = swtcf.dense_tn(A, B)
    torch.cuda.synchronize()
    assert rel_l2(C, A.double().t() @ B.double()) < REL


@pytest.mark.parametrize("M,N", [(100, 256), (256, 100)])
def test_dense_tn_strided_rows_and_accumulate(M, N):
    """Row strides above the width (a view of wider buffers, as the layer's
    AX view of denseC) and C += A^T B into a strided C, in both orientations
    (256 x 100 runs as C^T = B^T A)."""
    from tcc_amd import swtcf

    K = 9001
    A0, B0 = inputs(K, M + 28, N + 3, 5)
    A, B = A0[:, 3:3 + M], B0[:, :N]
    assert A.stride(0) == M + 28 and B.stride(0) == N + 3
    Cbig = torch.randn(M, N + 5, device="cuda")
    C = Cbig[:, :N]
    before = C.clone()
    extra = Cbig[:, N:].clone()
    swtcf.dense_tn(A, B, C, accumulate=True)
    torch.cuda.synchronize()
    want = before.double() + A.double().t() @ B.double()
    assert rel_l2(C, want) < REL
    assert torch.equal(Cbig[:, N:], extra)  # columns past N untouched
    swtcf.dense_tn(A, B, C)
    assert rel_l2(C, A.double().t() @ B.double()) < REL


def test_dense_tn_repeat_is_deterministic():
    """Partials are summed in a fixed order: two calls agree bit for bit."""
    from tcc_amd import swtcf

    A, B = inputs(300007, 100, 256, 11)
    C1 = swtcf.dense_tn(A, B)
    C2 = swtcf.dense_tn(A, B)
    torch.cuda.synchronize()
    assert torch.equal(C1, C2)


def test_dense_tn_empty_k():
    from tcc_amd import swtcf

    A = torch.empty((0, 7), device="cuda")
    B = torch.empty((0, 5), device="cuda")
    C = torch.full((7, 5), 3.0, device="cuda")
    swtcf.dense_tn(A, B, C, accumulate=True)
    assert torch.all(C == 3.0)
    swtcf.dense_tn(A, B, C)
    assert torch.all(C == 0.0)


def test_dense_tn_argument_errors():
    from tcc_amd import _lib

    L = _lib.lib()
    A = torch.randn(64, 10, device="cuda")
    B = torch.randn(64, 20, device="cuda")
    C = torch.empty(10, 20, device="cuda")
    need = L.tcc_dense_tn_workspace_bytes(64, 10, 20)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    # lda below M
    assert L.tcc_dense_tn(A.data_ptr(), 9, B.data_ptr(), 20, C.data_ptr(), 20, 64, 10, 20, 0, ws.data_ptr(), need,
                          None) == 1
    # workspace too small
    assert L.tcc_dense_tn(A.data_ptr(), 10, B.data_ptr(), 20, C.data_ptr(), 20, 64, 10, 20, 0, ws.data_ptr(),
                          need - 4, None) == 1
    assert b"workspace too small" in L.tcc_last_error()
    assert L.tcc_dense_tn(A.data_ptr(), 10, B.data_ptr(), 20, C.data_ptr(), 20, 64, 10, 20, 0, ws.data_ptr(), need,
                          None) == 0
    torch.cuda.synchronize()
    assert rel_l2(C, A.double().t() @ B.double()) < REL


RELU_SHAPES = [(64, 100, 256, 2), (50021, 100, 256, 2), (1999, 20, 48, 3), (3001, 130, 300, 8), (5, 7, 17, 1),
               (20000, 8, 40, 5), (4099, 257, 129, 2)]


@pytest.mark.parametrize("K,F,Hd,C", RELU_SHAPES)
def test_gcn_relu_grad_matches_float64(K, F, Hd, C):
    """dW1 = AXᵀ((G W2ᵀ) ⊙ [H > 0]) and dW2 = Hᵀ G against float64; H is a
    relu output (about half zeros)."""
    from tcc_amd import swtcf

    g = torch.Generator(device="cpu").manual_seed(K + 7 * F + 13 * Hd + C)
    AX = torch.randn(K, F, generator=g)
    H = torch.relu(torch.randn(K, Hd, generator=g))
    G = torch.randn(K, C, generator=g)
    W2 = torch.randn(Hd, C, generator=g)
    dW1, dW2 = swtcf.gcn_relu_grad(AX.cuda(), H.cuda(), G.cuda(), W2.cuda())
    torch.cuda.synchronize()
    d = (G.double() @ W2.double().t()) * (H > 0).double()
    assert rel_l2(dW1, AX.double().t() @ d) < REL
    assert rel_l2(dW2, H.double().t() @ G.double()) < REL


def test_gcn_relu_grad_strided_and_limits():
    from tcc_amd import _lib, swtcf

    K, F, Hd, C = 7001, 100, 256, 2
    g = torch.Generator(device="cpu").manual_seed(3)
    AXw = torch.randn(K, F + 4, generator=g).cuda()
    Hw = torch.relu(torch.randn(K, Hd + 8, generator=g)).cuda()
    Gw = torch.randn(K, C + 1, generator=g).cuda()
    W2 = torch.randn(Hd, C, generator=g).cuda()
    AX, H, G = AXw[:, :F], Hw[:, 8:], Gw[:, 1:]
    dW1, dW2 = swtcf.gcn_relu_grad(AX, H, G, W2)
    torch.cuda.synchronize()
    d = (G.double() @ W2.double().t()) * (H > 0).double()
    assert rel_l2(dW1, AX.double().t() @ d) < REL
    assert rel_l2(dW2, H.double().t() @ G.double()) < REL
    L = _lib.lib()
    W9 = torch.randn(Hd, 9, device="cuda")
    G9 = torch.randn(K, 9, device="cuda")
    out1 = torch.empty(F, Hd, device="cuda")
    out2 = torch.empty(Hd, 9, device="cuda")
    assert L.tcc_gcn_relu_grad(AX.data_ptr(), F + 4, H.data_ptr(), Hd + 8, G9.data_ptr(), 9, W9.data_ptr(),
                               out1.data_ptr(), out2.data_ptr(), K, F, Hd, 9, None, 0, None) == 3
    assert b"at most 8 classes" in L.tcc_last_error()


FWD_SHAPES = [(16, 100, 256, 2), (50021, 100, 256, 2), (1999, 20, 48, 3), (3001, 128, 200, 4), (5, 7, 17, 1),
              (20000, 64, 256, 2), (1, 1, 1, 1), (17, 113, 256, 4), (4093, 99, 256, 2)]


@pytest.mark.parametrize("K,F,Hd,C", FWD_SHAPES)
def test_gcn_relu_forward_matches_float64(K, F, Hd, C):
    """H = relu(AX W1) and XW = H W2 against float64 (F = 99, 113: the
    element-wise load path; F = 7: a partial input block)."""
    from tcc_amd import swtcf

    g = torch.Generator(device="cpu").manual_seed(K + 3 * F + 5 * Hd + C)
    AX = torch.randn(K, F, generator=g)
    W1 = torch.randn(F, Hd, generator=g) / F ** 0.5
    W2 = torch.randn(Hd, C, generator=g)
    H, XW = swtcf.gcn_relu_forward(AX.cuda(), W1.cuda(), W2.cuda())
    torch.cuda.synchronize()
    H64 = torch.relu(AX.double() @ W1.double())
    assert rel_l2(H, H64) < REL
    assert rel_l2(XW, H64 @ W2.double()) < REL


def test_gcn_relu_forward_strided_nan_and_limits():
    from tcc_amd import _lib, swtcf

    K, F, Hd, C = 3001, 100, 256, 2
    g = torch.Generator(device="cpu").manual_seed(9)
    AXw = torch.randn(K, F + 12, generator=g)
    AXw[77, 5] = float("nan")
    AX = AXw[:, 4:4 + F]
    W1 = torch.randn(F, Hd, generator=g) / 10
    W2 = torch.randn(Hd, C, generator=g)
    H, XW = swtcf.gcn_relu_forward(AX.cuda(), W1.cuda(), W2.cuda())
    torch.cuda.synchronize()
    H64 = torch.relu(AX.double() @ W1.double())
    ok = torch.ones(K, dtype=torch.bool)
    ok[77] = False
    assert rel_l2(H[ok.cuda()], H64[ok]) < REL
    assert rel_l2(XW[ok.cuda()], (H64 @ W2.double())[ok]) < REL
    # relu keeps NaN (torch.relu is clamp_min), as does H W2
    assert torch.isnan(H[77]).all() and torch.isnan(XW[77]).all()
    L = _lib.lib()
    X = torch.zeros(4, 129, device="cuda")
    w1 = torch.zeros(129, 8, device="cuda")
    w2 = torch.zeros(8, 2, device="cuda")
    h = torch.empty(4, 8, device="cuda")
    xw = torch.empty(4, 2, device="cuda")
    assert L.tcc_gcn_relu_forward(X.data_ptr(), 129, w1.data_ptr(), w2.data_ptr(), h.data_ptr(), 8, xw.data_ptr(), 2,
                                  4, 129, 8, 2, None) == 3
    assert b"F <= 128" in L.tcc_last_error()
