"""SAE-level entry points. `sae` is a saeflow_amd.SAE, or anything with the same
attributes (W_enc, b_enc, W_dec, b_dec, threshold, activation, k).

Mirrors saeflow/ops.py:12-49. Sparse features are CSR tuples (indptr, indices, values);
see kernels/decode.py.
"""

import torch

from .kernels import (dense_to_csr, encode_gather, encode_rows, exclusive_scan, fixed_width_to_dense, fused_encode,
                      overflow_rows, rows_to_csr, rows_topk, sparse_decode, topk_gather, topk_rows)

# Row-candidate paths: the fused encode appends each row's selected features to a per-row list
# instead of writing the dense [M, d_sae] features, which the reference writes and reads back
# (ops.py:13-14, 37-39). Rows whose list would exceed its capacity are encoded again on their
# own through the dense path and spliced into the result, so results never depend on the
# capacity and one long row costs a re-encode of that row, not of the batch.
ROW_PATHS = True   # False: always the dense path (the reference's structure)
ROW_CAP = 1024     # candidates per row for encode_sparse (relu / jumprelu)
TOPK_CAP = 4096    # candidates per row for TopK
TOPK_MIN_FEATURES = 16384  # TopK takes the row-candidate path from this dictionary size on
TOPK_REDO_BYTES = 1 << 31  # dense features of the overflowed rows redone per chunk (at least 256 rows)


def _topk_dense(sae, x):
    f = fused_encode(x, sae.W_enc, sae.b_enc, sae.b_dec, activation="relu")
    return topk_rows(f, sae.k)


def _floor_slice(N, k):
    """Features whose top-k floor bounds the row-candidate TopK: a multiple of 256, at least
    4096 and 8k."""
    S = min(N, max(4096, 8 * k))
    return (S + 255) // 256 * 256


def _topk_rows(sae, x):
    """TopK without the dense features: the k-th largest ReLU value over the first S features
    bounds each row's k-th largest value from below, so the fused encode keeps only values at
    or above it (about k * N / S per row, NaNs included) and the top-k of those lists is the
    top-k of the rows. Rows whose list overflowed are redone densely on the device: their ids
    and number stay in device memory, the gathered encode and top-k run over the live ones
    and replace those rows of the result, so, as the reference's TopK (ops.py:12-16), nothing
    is read back to the host. With no overflowed row the redo is a few near-empty launches."""
    M, N, k = x.shape[0], sae.W_enc.shape[1], sae.k
    S = _floor_slice(N, k)
    f_sub = fused_encode(x, sae.W_enc[:, :S], sae.b_enc[:S], sae.b_dec, activation="relu")
    floor = topk_rows(f_sub, k)[0][:, k - 1].float()
    del f_sub
    cnt, idx, val = encode_rows(x, sae.W_enc, sae.b_enc, sae.b_dec, activation="relu", cap=TOPK_CAP,
                                row_floor=floor)
    values, indices = rows_topk(cnt, idx, val, k, N)
    del idx, val
    rows, n_over = overflow_rows(cnt, TOPK_CAP)
    # the overflowed rows' dense features, in chunks of TOPK_REDO_BYTES or one 256-row block
    # (a single chunk at C4)
    chunk = min(M, max(256, TOPK_REDO_BYTES // (N * x.element_size()) // 256 * 256))
    for off in range(0, M, chunk):
        f = encode_gather(x, sae.W_enc, sae.b_enc, sae.b_dec, rows, n_over, row_off=off, out_rows=chunk)
        topk_gather(f, k, n_over, rows, values, indices, row_off=off)
        del f
    return values, indices


def _topk(sae, x):
    """ReLU fused encode, then the row top-k (ops.py:12-16): (values [M,k], indices int32 [M,k])."""
    N, k = sae.W_enc.shape[1], sae.k
    # the row path pays off when the floor slice is a small part of the row and the expected
    # list (k * N / S) sits well inside its capacity
    if (ROW_PATHS and x.shape[0] > 0 and N >= TOPK_MIN_FEATURES and 8 * k <= N // 4
            and k * N <= _floor_slice(N, k) * (TOPK_CAP // 2)):
        return _topk_rows(sae, x)
    return _topk_dense(sae, x)


def _fill_overflowed_rows(sae, x, cnt, indptr, indices, values):
    """CSR segments of the rows whose candidate list overflowed ROW_CAP: those rows alone are
    encoded densely (the same GEMM, so the same values and counts) and compacted, and each
    row's entries are copied into its segment of the batch's CSR."""
    over = torch.nonzero(cnt > ROW_CAP).flatten()
    row_nnz = torch.zeros(over.numel(), dtype=torch.int32, device=x.device)
    f = fused_encode(x[over], sae.W_enc, sae.b_enc, sae.b_dec, sae.threshold, sae.activation, row_nnz=row_nnz)
    sub_indptr, sub_indices, sub_values = dense_to_csr(f, row_nnz)
    del f
    n = sub_indices.numel()
    # entry e of over-row r goes to indptr[over[r]] + (e - sub_indptr[r])
    shift = torch.repeat_interleave(indptr[over] - sub_indptr[:-1], row_nnz.long(), output_size=n)
    pos = shift + torch.arange(n, device=x.device)
    indices[pos] = sub_indices
    values[pos] = sub_values


def _encode_sparse_rows(sae, x):
    """encode_sparse for relu / jumprelu through per-row candidate lists. The scan of the
    counts and its one host read (nnz, as dense_to_csr, decode.py:88) also bring back the
    longest list; rows longer than ROW_CAP are filled in by _fill_overflowed_rows."""
    cnt, idx, val = encode_rows(x, sae.W_enc, sae.b_enc, sae.b_dec, sae.threshold, sae.activation, cap=ROW_CAP)
    indptr = exclusive_scan(cnt)
    nnz, longest = torch.stack([indptr[-1], cnt.max().to(torch.int64)]).tolist()
    indices, values = rows_to_csr(cnt, idx, val, indptr, nnz)  # overflowed rows are skipped
    if longest > ROW_CAP:
        _fill_overflowed_rows(sae, x, cnt, indptr, indices, values)
    return indptr, indices, values


def encode(sae, x):
    """The features of every token as a dense [M, d_sae] tensor (ops.py:19-26)."""
    if sae.activation == "topk":
        values, indices = _topk(sae, x)
        return fixed_width_to_dense(indices, values, sae.W_enc.shape[1])
    return fused_encode(x, sae.W_enc, sae.b_enc, sae.b_dec, sae.threshold, sae.activation)


def encode_sparse(sae, x):
    """The features of every token in the CSR contract, (indptr int64 [M+1], indices int32
    [nnz], values [nnz]) (ops.py:29-39)."""
    M = x.shape[0]
    if sae.activation == "topk":
        # every row holds exactly k entries, so indptr is arange(0, M*k+1, k) and no scan or
        # compaction runs
        values, indices = _topk(sae, x)
        indptr = torch.arange(0, M * sae.k + 1, sae.k, device=x.device, dtype=torch.int64)
        return indptr, indices.flatten(), values.flatten()
    if ROW_PATHS and M > 0:
        return _encode_sparse_rows(sae, x)
    row_nnz = torch.zeros(M, device=x.device, dtype=torch.int32)
    f = fused_encode(x, sae.W_enc, sae.b_enc, sae.b_dec, sae.threshold, sae.activation, row_nnz=row_nnz)
    return dense_to_csr(f, row_nnz)


def decode_sparse(sae, csr):
    """x_hat [M, d_in] = b_dec + the W_dec rows the CSR selects, weighted by its values (ops.py:42-44)."""
    return sparse_decode(*csr, sae.W_dec, sae.b_dec)


def forward(sae, x):
    """decode_sparse(encode_sparse(x)) (ops.py:47-49): no dense [M, d_sae] tensor reaches the decoder."""
    return decode_sparse(sae, encode_sparse(sae, x))
