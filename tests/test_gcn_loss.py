"""gcn.cross_entropy against torch.nn.CrossEntropyLoss, the reference's loss
(train/tcgnn_conv_release.py:437), on the CPU: value and gradient, including
extreme logits (a log-sum-exp that would overflow exp) and one row."""
import pytest
import torch


@pytest.mark.parametrize("n,C,scale", [(1, 2, 1.0), (1000, 2, 1.0), (777, 47, 3.0), (64, 5, 200.0)])
def test_cross_entropy_matches_torch(n, C, scale):
    from tcc_amd import gcn

    g = torch.Generator().manual_seed(n * 10 + C)
    logits = (torch.randn(n, C, generator=g) * scale).requires_grad_(True)
    labels = torch.randint(0, C, (n,), generator=g)
    a = gcn.cross_entropy(logits, labels)
    (ga,) = torch.autograd.grad(a, logits)
    b = torch.nn.CrossEntropyLoss()(logits, labels)
    (gb,) = torch.autograd.grad(b, logits)
    assert torch.isfinite(a)
    assert torch.allclose(a, b, rtol=1e-6, atol=1e-6)
    assert torch.allclose(ga, gb, rtol=1e-5, atol=1e-8)
