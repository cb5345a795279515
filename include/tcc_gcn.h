/*
 * tcc_gcn.h — C-ABI of the dense products of the GCN layer backward on
 * MI355X (gfx950), beside the block-sparse SpMM of tcc_spmm_cnic.h.
 *
 * The weight gradient of a GCN layer is a tall-skinny transposed product
 * over all graph nodes:
 *   grad_weights = torch.mm(X_out.T, d_output)
 *     (TAC_training_backend/train/tcgnn_conv_release.py:150: X_out [n x F_in]
 *      is the aggregated input A·X, d_output [n x F_out])
 * and, for a layer evaluated as A·(X·W), grad_weights = X^T (A^T dY).  With n
 * in the millions and F in the hundreds, library GEMMs leave most of the
 * GPU idle on this shape; tcc_dense_tn splits the n rows over workgroups,
 * each accumulating its rows' product for a whole block of C with fp32
 * MFMA, and sums the partial products in a fixed order (deterministic).
 * Products and sums are fp32 (no TF32 rounding), as torch.mm in fp32.
 *
 * Errors as in tcc_swtcf.h: 0 or a TCC_ERR_* code, text in tcc_last_error().
 */
#ifndef TCC_GCN_H
#define TCC_GCN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Bytes of device workspace tcc_dense_tn needs for these sizes on the
 * current device (the split of K depends on its compute-unit count). */
size_t tcc_dense_tn_workspace_bytes(uint32_t K, uint32_t M, uint32_t N);

/* C[M x N] = A^T B (accumulate = 0) or C += A^T B (accumulate != 0), for
 * row-major A [K x M] with row stride lda >= M, B [K x N] with ldb >= N and
 * C with ldc >= N (strides in elements, below 2^28).  fp32 device pointers,
 * 4-byte aligned; `workspace` is device memory of at least
 * tcc_dense_tn_workspace_bytes(K, M, N) bytes, not shared with a concurrent
 * call.  Asynchronous on `stream` (a hipStream_t; NULL = the null stream).
 * Replaces torch.mm(X_out.T, d_output), tcgnn_conv_release.py:150. */
int tcc_dense_tn(const float* A, uint32_t lda, const float* B, uint32_t ldb, float* C, uint32_t ldc, uint32_t K,
                 uint32_t M, uint32_t N, int accumulate, void* workspace, size_t workspaceBytes, void* stream);

/* tcc_dense_tn without a workspace and without any allocation.  No
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory, such as code under HIP graph capture (a captured training
 * step) or a serving loop that forbids hipMalloc.  The partial products go
 * to a fixed device array inside the library, TCC_DENSE_TN_NOALLOC_SCRATCH_BYTES
 * (16 MiB) per GPU, held until the process ends; the split of K is capped so
 * that they fit (fewer splits than tcc_dense_tn picks only when its
 * workspace would exceed 16 MiB; the result is then the same up to fp32
 * summation order, else bit for bit).  Returns TCC_ERR_UNSUPPORTED when
 * M x N floats exceed the array.  Every call on a GPU shares that GPU's
 * array: calls that overlap on one GPU (on different streams, or from
 * different threads) race and must be serialised by the caller. */
#define TCC_DENSE_TN_NOALLOC_SCRATCH_BYTES (16u << 20)
int tcc_dense_tn_noalloc(const float* A, uint32_t lda, const float* B, uint32_t ldb, float* C, uint32_t ldc,
                         uint32_t K, uint32_t M, uint32_t N, int accumulate, void* stream);

/* H = relu(AX W1) [K x Hd] and XW = H W2 [K x C] in one pass over the K
 * rows of AX [K x F] (row strides ldax, ldh, ldxw; W1 [F x Hd] and W2
 * [Hd x C] row-major): the first layer's transform and activation and the
 * second layer's transform of a two-layer GCN, which the reference runs as
 * X_gat = torch.mm(X_out, weights) (train/tcgnn_conv_release.py:134),
 * self.relu (:231-238) and the last layer's torch.mm (:134 again) with H
 * written and read back in between.  fp32 MFMA products and sums; relu
 * keeps NaN (clamp_min).  F <= 128, Hd <= 256, C <= 4 (TCC_ERR_UNSUPPORTED
 * above).  No workspace. */
int tcc_gcn_relu_forward(const float* AX, uint32_t ldax, const float* W1, const float* W2, float* H, uint32_t ldh,
                         float* XW, uint32_t ldxw, uint32_t K, uint32_t F, uint32_t Hd, uint32_t C, void* stream);

/* Bytes of device workspace tcc_gcn_relu_grad needs (current device). */
size_t tcc_gcn_relu_grad_workspace_bytes(uint32_t K, uint32_t F, uint32_t Hd, uint32_t C);

/* Both weight gradients of a two-layer GCN, conv_final(relu(conv1(X))), in
 * one pass over the K node rows:
 *   dW1 [F x Hd] = AX^T ((G W2^T) (.) [H > 0])
 *   dW2 [Hd x C] = H^T G
 * with AX [K x F] the first layer's aggregated input (row stride ldax),
 * H [K x Hd] its relu output (ldh), G [K x C] = A^T dOut the second layer's
 * aggregated output gradient (ldg) and W2 [Hd x C] row-major, C <= 8
 * (TCC_ERR_UNSUPPORTED above).
 * This is what the reference's autograd runs as four steps
 * (train/tcgnn_conv_release.py:147-154 for each layer, with torch's relu
 * backward between): grad_X = grad_sp @ weights.T of the second layer,
 * the relu mask, and grad_weights = X_out.T @ d_output of both layers.
 * Products and sums in fp32; dW1 and dW2 are overwritten.  `workspace` as
 * for tcc_dense_tn, at least tcc_gcn_relu_grad_workspace_bytes bytes. */
int tcc_gcn_relu_grad(const float* AX, uint32_t ldax, const float* H, uint32_t ldh, const float* G, uint32_t ldg,
                      const float* W2, float* dW1, float* dW2, uint32_t K, uint32_t F, uint32_t Hd, uint32_t C,
                      void* workspace, size_t workspaceBytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TCC_GCN_H */
