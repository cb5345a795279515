"""Two-layer GCN step (tcc_amd.gcn, mirroring train/tcgnn_conv_release.py:49-250)
against a float64 numpy evaluation of the same formulas on a dense A:
  forward  AX = A·tf32(X) (the spmm_cnic mma.m16n8k8 numerics), out = AX·W
  backward dW = AXᵀ·dY, G = Aᵀ·dY in plain fp32 operands (torch.sparse.mm,
           :152), dX = G·Wᵀ
with a hot/cold feature table on the first layer.  Tolerance rel-L2 1e-4
(fp32 GEMMs on the GPU against fp64)."""
import numpy as np
import pytest
import torch

REL = 1e-4


def rel_l2(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


def tf32(a):
    b = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
    fin = (b & 0x7F800000) != 0x7F800000
    r = np.where(fin, (b + 0x1000) & 0xFFFFE000, b).astype(np.uint32)
    return r.view(np.float32).astype(np.float64)


def reference_step(A, X, W1, W2, labels, last_transform_first=True):
    """Forward/backward of the two-layer GCN in float64 with the kernels'
    rounding: TF32 operands into forward SpMMs, fp32 into the A^T product.
    The last layer (256 -> classes) runs A·(R·W2) as tcc_amd.gcn does, or
    (A·R)·W2 as the reference does (tcgnn_conv_release.py:133-134)."""
    AX1 = A @ tf32(X)
    H1 = AX1 @ W1
    R = np.maximum(H1, 0.0)
    if last_transform_first:
        out = A @ tf32((R @ W2).astype(np.float32))
    else:
        out = (A @ tf32(R.astype(np.float32))) @ W2
    m = out.max(axis=1, keepdims=True)
    logp = out - m - np.log(np.exp(out - m).sum(axis=1, keepdims=True))
    p = np.exp(logp)
    n = out.shape[0]
    loss = -np.mean(logp[np.arange(n), labels])
    dout = p.copy()
    dout[np.arange(n), labels] -= 1.0
    dout /= n
    G2 = A.T @ dout.astype(np.float32).astype(np.float64)
    dW2 = R.T @ G2  # = (A R)^T dout
    dR = G2 @ W2.T
    dH1 = dR * (H1 > 0)
    dW1 = AX1.T @ dH1
    return out, loss, dW1, dW2


@pytest.mark.gpu
@pytest.mark.parametrize("hot_fraction", [0.2, 0.0, 1.0])
def test_gcn_step_matches_dense_reference(gpu, hot_fraction):
    from tcc_amd import gcn
    from tcc_amd.graphs import rmat_graph

    n, F, H, C = 1999, 20, 48, 3
    rows, cols = rmat_graph(n, 25_000, 9)
    torch.manual_seed(0)
    X = torch.randn((n, F))
    table = gcn.FeatureTable(X, cols, hot_fraction=hot_fraction)
    g1, g2 = gcn.build_gcn_graphs(rows, cols, n, table.hot)
    model = gcn.GCN(F, H, C).cuda()
    labels = gcn.synthetic_labels(n, C, 1)
    W1 = model.conv1.weights.detach().cpu().numpy().astype(np.float64)
    W2 = model.conv_final.weights.detach().cpu().numpy().astype(np.float64)
    pred = model(g1, g2, table.source)
    loss = gcn.cross_entropy(pred, labels)
    loss.backward()
    torch.cuda.synchronize()
    A = np.zeros((n, n))
    A[rows.numpy(), cols.numpy()] = 1.0
    out, ref_loss, dW1, dW2 = reference_step(A, X.numpy(), W1, W2, labels.cpu().numpy())
    assert rel_l2(pred.detach().cpu().numpy(), out) < REL
    assert abs(loss.item() - ref_loss) < REL * abs(ref_loss)
    assert rel_l2(model.conv1.weights.grad.cpu().numpy(), dW1) < REL
    assert rel_l2(model.conv_final.weights.grad.cpu().numpy(), dW2) < REL
    # the reference's association order agrees to the north_star tolerance
    out_r, loss_r, dW1_r, dW2_r = reference_step(A, X.numpy(), W1, W2, labels.cpu().numpy(), False)
    assert rel_l2(pred.detach().cpu().numpy(), out_r) < 1e-3
    assert rel_l2(model.conv1.weights.grad.cpu().numpy(), dW1_r) < 1e-3
    assert rel_l2(model.conv_final.weights.grad.cpu().numpy(), dW2_r) < 1e-3
    table.free()


@pytest.mark.gpu
def test_fused_two_layer_matches_layer_by_layer(gpu):
    """TwoLayerFunction (one autograd node, fused weight gradients) against
    the layer-by-layer functions on the same weights: outputs and both
    weight gradients within fp32 rounding."""
    from tcc_amd import gcn
    from tcc_amd.graphs import rmat_graph

    n, F, H, C = 4093, 100, 256, 2
    rows, cols = rmat_graph(n, 60_000, 21)
    torch.manual_seed(2)
    X = torch.randn((n, F))
    table = gcn.FeatureTable(X, cols)
    g1, g2 = gcn.build_gcn_graphs(rows, cols, n, table.hot)
    model = gcn.GCN(F, H, C).cuda()
    labels = gcn.synthetic_labels(n, C, 4)
    res = []
    for fused in (True, False):
        model.fused = fused
        model.zero_grad(set_to_none=True)
        pred = model(g1, g2, table.source)
        gcn.cross_entropy(pred, labels).backward()
        res.append((pred.detach().clone(), model.conv1.weights.grad.clone(), model.conv_final.weights.grad.clone()))
    torch.cuda.synchronize()
    for a, b in zip(res[0], res[1]):
        assert rel_l2(a.cpu().numpy(), b.double().cpu().numpy()) < 1e-5
    table.free()


@pytest.mark.gpu
@pytest.mark.parametrize("F,H,C", [(150, 64, 3), (40, 256, 8), (32, 48, 12)])
def test_two_layer_paths_agree(gpu, F, H, C):
    """The paths GCN.forward picks besides the fully fused one, each against
    the layer-by-layer functions: F > 128 keeps torch's forward transform
    inside TwoLayerFunction (fused backward), 8 classes take the 8-wide
    relu-gradient tiles, 12 classes run layer by layer."""
    from tcc_amd import gcn
    from tcc_amd.graphs import rmat_graph

    n = 2039
    rows, cols = rmat_graph(n, 30_000, 23 + C)
    torch.manual_seed(C)
    X = torch.randn((n, F))
    table = gcn.FeatureTable(X, cols)
    g1, g2 = gcn.build_gcn_graphs(rows, cols, n, table.hot)
    model = gcn.GCN(F, H, C).cuda()
    labels = gcn.synthetic_labels(n, C, 5)
    res = []
    for fused in (True, False):
        model.fused = fused
        model.zero_grad(set_to_none=True)
        pred = model(g1, g2, table.source)
        gcn.cross_entropy(pred, labels).backward()
        res.append((pred.detach().clone(), model.conv1.weights.grad.clone(), model.conv_final.weights.grad.clone()))
    torch.cuda.synchronize()
    for a, b in zip(res[0], res[1]):
        assert rel_l2(a.cpu().numpy(), b.double().cpu().numpy()) < 1e-5
    table.free()


@pytest.mark.gpu
def test_packed_feature_table_gives_the_same_step(gpu):
    """FeatureTable(packed=True) holds TF32 rows packed in 2.5 bytes: the
    first layer rounds X to TF32 anyway, so the step agrees with the fp32
    table (up to the atomics' summation order)."""
    from tcc_amd import gcn
    from tcc_amd.graphs import rmat_graph

    n, F = 3001, 100
    rows, cols = rmat_graph(n, 40_000, 41)
    torch.manual_seed(4)
    X = torch.randn((n, F))
    res = []
    for packed in (False, True):
        table = gcn.FeatureTable(X, cols, packed=packed)
        g1, g2 = gcn.build_gcn_graphs(rows, cols, n, table.hot)
        torch.manual_seed(5)
        model = gcn.GCN(F, 64, 2).cuda()
        labels = gcn.synthetic_labels(n, 2, 7)
        pred = model(g1, g2, table.source)
        gcn.cross_entropy(pred, labels).backward()
        torch.cuda.synchronize()
        res.append((pred.detach().cpu(), model.conv1.weights.grad.cpu(), model.conv_final.weights.grad.cpu()))
        table.free()
    for a, b in zip(res[0], res[1]):
        assert rel_l2(a.numpy(), b.double().numpy()) < 1e-5


@pytest.mark.gpu
def test_dropout_takes_the_layer_path(gpu):
    """With dropout in training the model runs layer by layer (the mask sits
    between the layers); in eval mode dropout is the identity and the fused
    node runs: both give finite outputs and gradients."""
    from tcc_amd import gcn
    from tcc_amd.graphs import rmat_graph

    n, F = 1500, 24
    rows, cols = rmat_graph(n, 15_000, 31)
    torch.manual_seed(3)
    X = torch.randn((n, F))
    table = gcn.FeatureTable(X, cols)
    g1, g2 = gcn.build_gcn_graphs(rows, cols, n, table.hot)
    model = gcn.GCN(F, 32, 2, dropout=0.5).cuda()
    labels = gcn.synthetic_labels(n, 2, 6)
    for train in (True, False):
        model.train(train)
        model.zero_grad(set_to_none=True)
        loss = gcn.cross_entropy(model(g1, g2, table.source), labels)
        loss.backward()
        assert torch.isfinite(loss)
        assert torch.isfinite(model.conv1.weights.grad).all()
        assert torch.isfinite(model.conv_final.weights.grad).all()
    table.free()


@pytest.mark.gpu
def test_gcn_trains(gpu):
    """A few Adam steps on a small graph lower the loss (the full training
    step of tcgnn_conv_release.py:284-329)."""
    from tcc_amd import gcn
    from tcc_amd.graphs import rmat_graph

    n, F = 3000, 16
    rows, cols = rmat_graph(n, 30_000, 10)
    torch.manual_seed(1)
    X = torch.randn((n, F))
    table = gcn.FeatureTable(X, cols)
    g1, g2 = gcn.build_gcn_graphs(rows, cols, n, table.hot)
    model = gcn.GCN(F, 64, 2).cuda()
    labels = gcn.synthetic_labels(n, 2, 3)
    opt = torch.optim.Adam(model.parameters(), lr=0.003)
    losses = [gcn.train_epoch(model, g1, g2, table.source, labels, opt).item() for _ in range(30)]
    assert losses[-1] < losses[0]
    table.free()
