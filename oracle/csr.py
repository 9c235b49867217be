"""Bit-level CSR restatement in numpy — test infrastructure (see oracle/__init__.py).

Values are handled as raw bit patterns (uint16 for bf16/fp16, uint32 for fp32), so the
dense -> CSR result is exact for every dtype; an element is nonzero iff its magnitude bits
are nonzero, i.e. `f != 0.0` on the stored value (decode.py:70, encode.py:90).
"""

import numpy as np
import torch

_BITS = {torch.float64: (torch.int64, np.uint64, 0x7FFFFFFFFFFFFFFF),
         torch.float32: (torch.int32, np.uint32, 0x7FFFFFFF),
         torch.bfloat16: (torch.int16, np.uint16, 0x7FFF),
         torch.float16: (torch.int16, np.uint16, 0x7FFF)}


def to_bits(t):
    """torch float tensor -> numpy unsigned bit patterns of the same shape."""
    view_dt, np_dt, _ = _BITS[t.dtype]
    return t.detach().cpu().contiguous().view(view_dt).numpy().view(np_dt)


def from_bits(a, dtype):
    """numpy bit patterns -> torch tensor of `dtype`."""
    view_dt, np_dt, _ = _BITS[dtype]
    signed = {np.uint64: np.int64, np.uint32: np.int32, np.uint16: np.int16}[np_dt]
    return torch.from_numpy(np.ascontiguousarray(a).astype(np_dt).view(signed)).view(view_dt).view(dtype)


def dense_to_csr_bits(bits, mag_mask):
    """Canonical CSR of a [M, N] bit array (decode.py:77-94 with _compact_kernel :61-74):
    indptr int64 [M+1] = [0, cumsum(row nonzero counts)], indices int32 in increasing column
    order per row, values = the nonzero elements' bits."""
    bits = np.asarray(bits)
    nz = (bits & mag_mask) != 0
    counts = nz.sum(axis=1, dtype=np.int64)
    indptr = np.zeros(bits.shape[0] + 1, dtype=np.int64)
    np.cumsum(counts, out=indptr[1:])
    rows, cols = np.nonzero(nz)  # row-major scan: columns ascend within each row
    return indptr, cols.astype(np.int32), bits[rows, cols]


def dense_to_csr(f):
    """torch dense [M, N] -> (indptr int64, indices int32, values torch tensor of f.dtype)."""
    _, _, mask = _BITS[f.dtype]
    indptr, indices, vbits = dense_to_csr_bits(to_bits(f), mask)
    return indptr, indices, from_bits(vbits, f.dtype)


def row_counts(f):
    """Per-row nonzero counts of a torch tensor (the row_nnz invariant, test_kernels.py:44)."""
    _, _, mask = _BITS[f.dtype]
    return ((to_bits(f) & mask) != 0).sum(axis=1).astype(np.int64)


def csr_to_dense(indptr, indices, values, d_sae):
    """float64 dense [M, d_sae] from CSR, duplicate columns summed (decode.py:123-126)."""
    indptr = np.asarray(indptr, dtype=np.int64)
    M = indptr.size - 1
    out = np.zeros((M, d_sae), dtype=np.float64)
    vals = np.asarray(values, dtype=np.float64)
    idx = np.asarray(indices, dtype=np.int64)
    rows = np.repeat(np.arange(M), np.diff(indptr))
    np.add.at(out, (rows, idx), vals)
    return out


def sparse_decode(indptr, indices, values, W_dec, b_dec=None):
    """x_hat[m] = b_dec + sum_{j in row m} values[j] * W_dec[indices[j]] in float64
    (decode.py:28-55; the kernel's per-row gather, :42-51, and bias, :53-54)."""
    indptr = np.asarray(indptr, dtype=np.int64)
    W = np.asarray(W_dec, dtype=np.float64)
    vals = np.asarray(values, dtype=np.float64)
    idx = np.asarray(indices, dtype=np.int64)
    M = indptr.size - 1
    contrib = vals[:, None] * W[idx]
    out = np.zeros((M, W.shape[1]), dtype=np.float64)
    rows = np.repeat(np.arange(M), np.diff(indptr))
    np.add.at(out, rows, contrib)
    if b_dec is not None:
        out += np.asarray(b_dec, dtype=np.float64)[None, :]
    return out


def topk_rows(f, k):
    """Row top-k (ops.py:16, f.topk(k, dim=-1)) with the tie rule made explicit: values
    descending as torch.topk compares them (-0.0 equals +0.0; NaN, of either sign, ranks
    above every number and all NaNs are equal), equal values by increasing column.
    f: float array [M, N] -> (values, cols)."""
    f = np.asarray(f, dtype=np.float64)
    M, N = f.shape
    cols = np.broadcast_to(np.arange(N), f.shape)
    nan = np.isnan(f)
    order = np.lexsort((cols, -np.where(nan, 0.0, f), ~nan), axis=1)[:, :k]
    return np.take_along_axis(f, order, axis=1), order.astype(np.int32)
