"""Two-layer GCN on the block-sparse SpMM: the caller of the hot path
(train/tcgnn_conv_release.py:49-250), on MI355X.

CNICSPMMFunction mirrors the reference's autograd function
(tcgnn_conv_release.py:49-166):
  forward : AX = A·X with the spmm_cnic split (BCSR part + BCSC part,
            spmm_launcher.cu:30-271), out = AX·W                (:130-134)
  backward: dW = AXᵀ·dY, G = Aᵀ·dY, dX = G·Wᵀ                    (:147-154)
The weight gradients AXᵀ·dY and Xᵀ·G are tall-skinny products over all nodes
(tcc_dense_tn: K split over workgroups on fp32 MFMA), where library GEMMs
reach a fraction of the GPU on this shape.
The reference's G = torch.sparse.mm(Aᵀ, dY) over unit values (:139-142, :152)
is the block-sparse transposed gather over a BCSC of the whole A
(tcc_bcsc_transpose_spmm), and dX is computed only when the layer's input
needs a gradient (the reference computes and discards it for the first
layer, whose input is the feature table).

A later layer whose output is narrower than its input (the last layer:
256 -> 2 classes) is evaluated as A·(X·W) instead of (A·X)·W — the same
product in exact arithmetic, with the SpMM at the output width and the
backward G = Aᵀ·dY, dW = Xᵀ·G, dX = G·Wᵀ (the aggregate-then-transform order
of :133-134 would gather 256-wide rows for a 2-wide result).

The first layer reads X through the hot/cold feature source of
spmm_kernel.cu:129-153: edges whose source row is hot (in the HBM feature
cache) go to the BCSR gather, edges with cold sources to the BCSC scatter,
which reads each cold row once per column window from mapped pinned host
memory.  Later layers read device-resident X and put every edge in the
BCSR gather.

GCN = conv1 (first layer, F_in -> hidden), ReLU, dropout, conv_final
(hidden -> classes), weights xavier-uniform (tcgnn_conv_release.py:168-250);
trained with cross-entropy and Adam (:448-449).  Without dropout and with at
most 8 classes the two layers run as one autograd node whose backward forms
both weight gradients in one pass (TwoLayerFunction).
"""
from __future__ import annotations

import numpy as np
import torch

from . import swtcf
from .hostmem import PinnedArray


class LayerGraph:
    """The block matrices of one layer's A [num_rows x num_cols]:
    forward BCSR (edges whose source is on the device) and BCSC (edges whose
    source is cold, or None), and the backward BCSC of every edge (shared
    between layers over the same A)."""

    def __init__(self, rows: torch.Tensor, cols: torch.Tensor, num_rows: int, num_cols: int,
                 hot_src: torch.Tensor | None = None, backward_bcsc: swtcf.BlockMatrix | None = None):
        rows, cols = rows.cuda(), cols.cuda()
        r = rows.to(torch.int32).contiguous()
        c = cols.to(torch.int32).contiguous()
        self.num_rows, self.num_cols = num_rows, num_cols
        if hot_src is None:
            self.bcsr = swtcf.coo_to_bcsr(r, c, None, num_rows, num_cols)
            self.bcsc = None
        else:
            h = hot_src[cols.long()]
            self.bcsr = _bcsr_or_empty(r[h].contiguous(), c[h].contiguous(), num_rows, num_cols)
            self.bcsc = _bcsc_or_empty(r[~h].contiguous(), c[~h].contiguous(), num_rows, num_cols)
        self.bwd = backward_bcsc if backward_bcsc is not None else swtcf.coo_to_bcsc(r, c, None, num_rows, num_cols)

    def aggregate(self, F: int, x: torch.Tensor | None = None, source=None) -> torch.Tensor:
        """AX [num_rows x F] (a view of the (RW+1)*8-row denseC buffer)."""
        RW = self.bcsr.view.num_rowWindows
        denseC = torch.empty(((RW + 1) * 8, F), dtype=torch.float32, device="cuda")
        if source is not None:
            bcsc = self.bcsc if self.bcsc is not None else _EMPTY_BCSC
            swtcf.spmm_cnic_forward_mixed(self.bcsr, bcsc, source, denseC, F)
        elif self.bcsc is not None:
            swtcf.spmm_cnic_forward(self.bcsr, self.bcsc, x, denseC)
        else:
            denseC[RW * 8:].zero_()
            swtcf.bcsr_spmm(self.bcsr, x, denseC[: RW * 8])
        return denseC[: self.num_rows]

    def transpose_aggregate(self, dY: torch.Tensor) -> torch.Tensor:
        """Aᵀ dY [num_cols x F]."""
        out = swtcf.bcsc_transpose_spmm(self.bwd, dY.contiguous())
        return out[: self.num_cols]


def _bcsr_or_empty(r, c, num_rows, num_cols):
    if r.numel() > 0:
        return swtcf.coo_to_bcsr(r, c, None, num_rows, num_cols)
    RW = (num_rows + 7) // 8
    keep = (torch.zeros(RW + 1, dtype=torch.int32, device="cuda"), torch.zeros(1, dtype=torch.int32, device="cuda"),
            torch.full((8,), -1, dtype=torch.int32, device="cuda"), torch.zeros(1, dtype=torch.int64, device="cuda"))
    return swtcf.wrap_bcsr(num_rows, num_cols, 0, 0, RW, *keep)


def _bcsc_or_empty(r, c, num_rows, num_cols):
    if r.numel() > 0:
        return swtcf.coo_to_bcsc(r, c, None, num_rows, num_cols)
    return _EMPTY_BCSC


class _EmptyBCSC:
    view = swtcf.BCSC()  # no windows: the scatter launches nothing


_EMPTY_BCSC = _EmptyBCSC()


class CNICSPMMFunction(torch.autograd.Function):
    """out = (A X) W with the reference's backward (tcgnn_conv_release.py:49-166)."""

    @staticmethod
    def forward(ctx, graph: LayerGraph, source, x, weights):
        F = weights.shape[0]
        AX = graph.aggregate(F, x=None if source is not None else x.contiguous(), source=source)
        ctx.graph = graph
        ctx.save_for_backward(AX, weights)
        return torch.mm(AX, weights)

    @staticmethod
    def backward(ctx, d_output):
        AX, weights = ctx.saved_tensors
        grad_weights = swtcf.dense_tn(AX, d_output)  # AXᵀ·dY (:150)
        grad_x = None
        if ctx.needs_input_grad[2]:
            grad_sp = ctx.graph.transpose_aggregate(d_output)
            grad_x = torch.mm(grad_sp, weights.t())
        return None, None, grad_x, grad_weights


class TransformFirstFunction(torch.autograd.Function):
    """out = A (X W), the same product as (A X) W associated the other way,
    for layers whose output is narrower than their input: the SpMM then runs
    at the output width (2 instead of 256 for the GCN's last layer).
    Backward: G = Aᵀ dY (needed for dX in either order), dW = Xᵀ G,
    dX = G Wᵀ — AX is never formed."""

    @staticmethod
    def forward(ctx, graph: LayerGraph, x, weights):
        xw = torch.mm(x, weights).contiguous()
        out = graph.aggregate(weights.shape[1], x=xw)
        ctx.graph = graph
        ctx.save_for_backward(x, weights)
        return out

    @staticmethod
    def backward(ctx, d_output):
        x, weights = ctx.saved_tensors
        grad_sp = ctx.graph.transpose_aggregate(d_output)
        grad_weights = swtcf.dense_tn(x, grad_sp)  # Xᵀ·G
        grad_x = torch.mm(grad_sp, weights.t()) if ctx.needs_input_grad[1] else None
        return None, grad_x, grad_weights


class GCNConv(torch.nn.Module):
    def __init__(self, input_dim: int, output_dim: int, first_layer: bool = False):
        super().__init__()
        self.first_layer = first_layer
        self.weights = torch.nn.Parameter(torch.empty(input_dim, output_dim))
        torch.nn.init.xavier_uniform_(self.weights)

    def forward(self, graph: LayerGraph, source=None, x: torch.Tensor | None = None) -> torch.Tensor:
        in_dim, out_dim = self.weights.shape
        if not self.first_layer and out_dim < in_dim:
            # A(XW) = (AX)W: aggregate at the narrower width
            return TransformFirstFunction.apply(graph, x, self.weights)
        return CNICSPMMFunction.apply(graph, source if self.first_layer else None, x, self.weights)


class TwoLayerFunction(torch.autograd.Function):
    """conv_final(relu(conv1(X))) as one autograd node, for a last layer
    narrower than the hidden one and no dropout (what the layer-by-layer
    functions compute, with the backward fused):
      forward : AX = A X (first-layer source), then H = relu(AX W1) and
                XW = H W2 in one pass (tcc_gcn_relu_forward, F <= 128,
                hidden <= 256, classes <= 4), out = A XW
      backward: G = Aᵀ dOut, then one pass over AX, H and G for
                dW1 = AXᵀ((G W2ᵀ) ⊙ [H > 0]) and dW2 = Hᵀ G
                (tcc_gcn_relu_grad): G W2ᵀ, the relu mask and the hidden
                gradient are never written to memory."""

    @staticmethod
    def forward(ctx, g1: LayerGraph, g2: LayerGraph, source, w1, w2):
        AX = g1.aggregate(w1.shape[0], source=source)
        if swtcf.gcn_relu_forward_supported(w1.shape[0], w1.shape[1], w2.shape[1]):
            H, XW = swtcf.gcn_relu_forward(AX, w1, w2)  # one pass, H written once
        else:
            H = torch.relu(torch.mm(AX, w1))
            XW = torch.mm(H, w2).contiguous()
        out = g2.aggregate(w2.shape[1], x=XW)
        ctx.g2 = g2
        ctx.save_for_backward(AX, H, w2)
        return out

    @staticmethod
    def backward(ctx, d_output):
        AX, H, w2 = ctx.saved_tensors
        G = ctx.g2.transpose_aggregate(d_output)
        dw1, dw2 = swtcf.gcn_relu_grad(AX, H, G, w2)
        return None, None, None, dw1, dw2


# Class counts the fused two-layer backward takes (tcc_gcn_relu_grad).
FUSED_MAX_CLASSES = 8


class GCN(torch.nn.Module):
    def __init__(self, num_features: int, hidden_dim: int, num_classes: int, dropout: float = 0.0,
                 fused: bool = True):
        super().__init__()
        self.conv1 = GCNConv(num_features, hidden_dim, first_layer=True)
        self.conv_final = GCNConv(hidden_dim, num_classes)
        self.dropout = torch.nn.Dropout(p=dropout)
        self.fused = fused

    def forward(self, g1: LayerGraph, g2: LayerGraph, source) -> torch.Tensor:
        w1, w2 = self.conv1.weights, self.conv_final.weights
        no_dropout = self.dropout.p == 0.0 or not self.training
        if self.fused and no_dropout and w2.shape[1] < w2.shape[0] and w2.shape[1] <= FUSED_MAX_CLASSES:
            return TwoLayerFunction.apply(g1, g2, source, w1, w2)
        x = torch.relu(self.conv1(g1, source=source))
        x = self.dropout(x)
        return self.conv_final(g2, x=x)


class FeatureTable:
    """Features of every node: the hot rows (top `hot_fraction` of nodes by
    in-degree as a source, ties by id) in an HBM cache, all rows in mapped
    pinned host memory, and the tcc_feature_source that resolves them
    (cache_search_map = hot rank or -1, id_map = identity).

    packed=True stores both tables as TF32 rows packed by tcc_tf32_pack: the
    first layer's products round X to TF32 anyway, so they are the same bit
    for bit, and a cold row crosses the host link in 2.5 instead of 4 bytes
    per feature.  The default keeps the reference's fp32 rows."""

    def __init__(self, X: torch.Tensor, cols: torch.Tensor, hot_fraction: float = 0.2, packed: bool = False):
        n, F = X.shape
        deg = torch.bincount(cols.long().cuda(), minlength=n)
        n_hot = max(1, int(round(n * hot_fraction)))
        # degree descending, id ascending: sort by (-deg, id) through a stable sort
        order = torch.sort(-deg, stable=True).indices
        hot_ids = torch.sort(order[:n_hot]).values
        self.hot = torch.zeros(n, dtype=torch.bool, device="cuda")
        self.hot[hot_ids] = True
        csm = torch.full((n,), -1, dtype=torch.int32, device="cuda")
        csm[hot_ids] = torch.arange(n_hot, dtype=torch.int32, device="cuda")
        Xd = X.cuda()
        if packed:
            self.cache = swtcf.tf32_pack(Xd[hot_ids].contiguous())
            rows = swtcf.tf32_pack(Xd)
            self.host = PinnedArray((rows.numel(),), dtype=np.uint8)
            self.host.array[:] = rows.cpu().numpy()
            del rows
        else:
            self.cache = Xd[hot_ids].contiguous()
            self.host = PinnedArray((n, F))
            self.host.array[:] = X.cpu().numpy()
        del Xd
        self.ptrs = torch.tensor([self.cache.data_ptr()], dtype=torch.int64, device="cuda")
        self.ids = torch.arange(n, dtype=torch.int32, device="cuda")
        self.csm = csm
        fmt = swtcf.ROWS_TF32_PACKED if packed else swtcf.ROWS_FP32
        self.device_error = torch.zeros(1, dtype=torch.int32, device="cuda")
        self.source = swtcf.feature_source(self.ids, csm, self.ptrs, n_hot, self.host.device_ptr, n * F, fmt,
                                           device_error=self.device_error)
        self.n_hot = n_hot
        self.packed = packed

    def error(self) -> int:
        """TCC_DEVERR_FEATURE_INDEX if a lookup fell outside the tables since
        the last call (or since the table was made), else 0; synchronises
        the device and clears the word, as spmm_cnic.feature_error does."""
        v = int(self.device_error.item())
        self.device_error.zero_()
        return v

    def free(self) -> None:
        self.host.free()


def build_gcn_graphs(rows: torch.Tensor, cols: torch.Tensor, n: int, hot: torch.Tensor):
    """(first-layer graph with the hot/cold split, later-layer graph), both
    over the same A, sharing the backward BCSC."""
    g2 = LayerGraph(rows, cols, n, n)
    g1 = LayerGraph(rows, cols, n, n, hot_src=hot, backward_bcsc=g2.bwd)
    return g1, g2


def cross_entropy(pred: torch.Tensor, labels: torch.Tensor) -> torch.Tensor:
    """Mean cross-entropy of logits [n x C] against class ids: the value and
    gradient of torch.nn.CrossEntropyLoss() (tcgnn_conv_release.py:437),
    evaluated as log_softmax, gather and mean.  torch's 2-D nll_loss with mean
    reduction runs its forward and backward in one workgroup (2.2 ms and
    1.1 ms for 2.45M rows on MI355X); these run across the GPU."""
    return -torch.log_softmax(pred, dim=1).gather(1, labels.view(-1, 1)).mean()


def train_epoch(model: GCN, g1: LayerGraph, g2: LayerGraph, source, labels: torch.Tensor,
                optimizer: torch.optim.Optimizer, loss_fcn=cross_entropy) -> torch.Tensor:
    """One full-graph step: forward, loss, backward, optimizer step
    (train_one_step, tcgnn_conv_release.py:284-329)."""
    pred = model(g1, g2, source)
    loss = loss_fcn(pred, labels)
    optimizer.zero_grad()
    loss.backward()
    optimizer.step()
    return loss


def synthetic_labels(n: int, num_classes: int, seed: int) -> torch.Tensor:
    g = torch.Generator(device="cpu").manual_seed(seed + 2000)
    return torch.randint(0, num_classes, (n,), generator=g).cuda()

