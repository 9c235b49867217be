"""SAE-level entry points. `sae` is a saeflow_amd.SAE, or anything with the same
attributes (W_enc, b_enc, W_dec, b_dec, threshold, activation, k).

Mirrors saeflow/ops.py:12-49. Sparse features are CSR tuples (indptr, indices, values);
see kernels/decode.py.
"""

import torch

from .kernels import (dense_to_csr, encode_rows, exclusive_scan, fixed_width_to_dense, fused_encode, rows_to_csr,
                      rows_topk, sparse_decode, topk_rows)

# Row-candidate paths: the fused encode appends each row's selected features to a per-row list
# instead of writing the dense [M, d_sae] features, which the reference writes and reads back
# (ops.py:13-14, 37-39). A row whose list would exceed its capacity sends the whole call down
# the dense path, so results never depend on the capacity.
ROW_PATHS = True   # False: always the dense path (the reference's structure)
ROW_CAP = 1024     # candidates per row for encode_sparse (relu / jumprelu)
TOPK_CAP = 4096    # candidates per row for TopK
TOPK_MIN_FEATURES = 16384  # TopK takes the row-candidate path from this dictionary size on


def _topk_dense(sae, x):
    f = fused_encode(x, sae.W_enc, sae.b_enc, sae.b_dec, activation="relu")
    return topk_rows(f, sae.k)


def _topk_rows(sae, x):
    """TopK without the dense features: the k-th largest ReLU value over the first S features
    bounds each row's k-th largest value from below, so the fused encode keeps only values at
    or above it (about k * N / S per row) and the top-k of those lists is the top-k of the
    rows. Returns None when a list overflowed (one int read back to check)."""
    N, k = sae.W_enc.shape[1], sae.k
    S = min(N, max(4096, 8 * k))
    S = (S + 255) // 256 * 256
    f_sub = fused_encode(x, sae.W_enc[:, :S], sae.b_enc[:S], sae.b_dec, activation="relu")
    floor = topk_rows(f_sub, k)[0][:, k - 1].float()
    del f_sub
    cnt, idx, val = encode_rows(x, sae.W_enc, sae.b_enc, sae.b_dec, activation="relu", cap=TOPK_CAP,
                                row_floor=floor)
    top = rows_topk(cnt, idx, val, k, N)  # queued before the host read, so no launch gap
    if int(cnt.max()) > TOPK_CAP:
        return None
    return top


def _topk(sae, x):
    """ReLU fused encode, then the row top-k (ops.py:12-16): (values [M,k], indices int32 [M,k])."""
    N = sae.W_enc.shape[1]
    if ROW_PATHS and x.shape[0] > 0 and N >= TOPK_MIN_FEATURES and 8 * sae.k <= N // 4:
        top = _topk_rows(sae, x)
        if top is not None:
            return top
    return _topk_dense(sae, x)


def _encode_sparse_rows(sae, x):
    """encode_sparse for relu / jumprelu through per-row candidate lists; None when a list
    overflowed. The scan of the counts and its one host read (nnz, as dense_to_csr,
    decode.py:88) also bring back the longest list."""
    cnt, idx, val = encode_rows(x, sae.W_enc, sae.b_enc, sae.b_dec, sae.threshold, sae.activation, cap=ROW_CAP)
    indptr = exclusive_scan(cnt)
    nnz, longest = torch.stack([indptr[-1], cnt.max().to(torch.int64)]).tolist()
    if longest > ROW_CAP:
        return None
    indices, values = rows_to_csr(cnt, idx, val, indptr, nnz)
    return indptr, indices, values


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
    if ROW_PATHS and M > 0:
        csr = _encode_sparse_rows(sae, x)
        if csr is not None:
            return csr
    row_nnz = torch.zeros(M, device=x.device, dtype=torch.int32)
    f = fused_encode(x, sae.W_enc, sae.b_enc, sae.b_dec, sae.threshold, sae.activation, row_nnz=row_nnz)
    return dense_to_csr(f, row_nnz)


def decode_sparse(sae, csr):
    """Reconstruction [M, d_in] from CSR features."""
    return sparse_decode(*csr, sae.W_dec, sae.b_dec)


def forward(sae, x):
    """encode_sparse then decode_sparse: the dense feature matrix never reaches the decoder."""
    return decode_sparse(sae, encode_sparse(sae, x))
