"""SAE-level entry points. `sae` is a saeflow_amd.SAE, or anything with the same
attributes (W_enc, b_enc, W_dec, b_dec, threshold, activation, k).

Mirrors saeflow/ops.py:12-49. Sparse features are CSR tuples (indptr, indices, values);
see kernels/decode.py.
"""

import torch

from .kernels import dense_to_csr, fixed_width_to_dense, fused_encode, sparse_decode, topk_rows


def _topk(sae, x):
    """ReLU fused encode, then the row top-k (ops.py:12-16): (values [M,k], indices int32 [M,k])."""
    f = fused_encode(x, sae.W_enc, sae.b_enc, sae.b_dec, activation="relu")
    return topk_rows(f, sae.k)


def encode(sae, x):
    """Dense feature activations [M, d_sae]."""
    if sae.activation == "topk":
        values, indices = _topk(sae, x)
        return fixed_width_to_dense(indices, values, sae.W_enc.shape[1])
    return fused_encode(x, sae.W_enc, sae.b_enc, sae.b_dec, sae.threshold, sae.activation)


def encode_sparse(sae, x):
    """Feature activations as CSR (indptr, indices, values)."""
    M = x.shape[0]
    if sae.activation == "topk":
        # TopK is fixed-width already: no compaction pass needed.
        values, indices = _topk(sae, x)
        indptr = torch.arange(0, M * sae.k + 1, sae.k, device=x.device, dtype=torch.int64)
        return indptr, indices.flatten(), values.flatten()
    row_nnz = torch.zeros(M, device=x.device, dtype=torch.int32)
    f = fused_encode(x, sae.W_enc, sae.b_enc, sae.b_dec, sae.threshold, sae.activation, row_nnz=row_nnz)
    return dense_to_csr(f, row_nnz)


def decode_sparse(sae, csr):
    """Reconstruction [M, d_in] from CSR features."""
    return sparse_decode(*csr, sae.W_dec, sae.b_dec)


def forward(sae, x):
    """encode_sparse then decode_sparse: the dense feature matrix never reaches the decoder."""
    return decode_sparse(sae, encode_sparse(sae, x))
