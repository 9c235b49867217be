"""Sparse SAE decode, the dense -> CSR conversion and the row top-k, on gfx950.

Features travel as CSR: token m owns the entries indptr[m] .. indptr[m+1]-1 of `indices`
(feature ids, int32) and `values` (the feature dtype); indptr is int64 [M+1]. The decode
sums, per token, b_dec plus its features' W_dec rows scaled by their values, so it touches
only the L0 rows of W_dec a token uses. Mirrors saeflow/kernels/decode.py:77-126
(dense_to_csr, sparse_decode, csr_to_dense): same signatures, defaults and results.
"""

import ctypes

import torch

from .. import _lib


def row_counts(f):
    """int32 [M] nonzero counts of the rows of f [M, N] (torch.count_nonzero(f, dim=1), decode.py:85)."""
    M, N = f.shape
    dev = _lib.require_gpu(("f", f))
    counts = torch.empty(M, dtype=torch.int32, device=f.device)
    if M:
        with torch.cuda.device(dev):
            _lib.check(_lib.load().sf_count_nonzero(_lib.ptr(f), f.stride(0), f.stride(1), _lib.dtype_code(f, "f"),
                                                    M, N, _lib.ptr(counts), _lib.stream(dev)))
    return counts


def exclusive_scan(row_nnz):
    """indptr int64 [M+1] = [0, cumsum(row_nnz)] (decode.py:86-87); row_nnz int32 [M] on the GPU."""
    M = row_nnz.numel()
    dev = _lib.require_gpu(("row_nnz", row_nnz))
    row_nnz = row_nnz.reshape(M).to(torch.int32).contiguous()
    indptr = torch.empty(M + 1, dtype=torch.int64, device=row_nnz.device)
    with torch.cuda.device(dev):
        _lib.check(_lib.load().sf_scan_counts(_lib.ptr(row_nnz), M, _lib.ptr(indptr), _lib.stream(dev)))
    return indptr


def compact(f, indptr, nnz):
    """(indices int32 [nnz], values [nnz]): the nonzeros of every row of f in column order,
    placed at indptr[row] (_compact_kernel, decode.py:61-74)."""
    M, N = f.shape
    dev = _lib.require_gpu(("f", f), ("indptr", indptr))
    indices = torch.empty(nnz, dtype=torch.int32, device=f.device)
    values = torch.empty(nnz, dtype=f.dtype, device=f.device)
    if nnz and M:
        with torch.cuda.device(dev):
            _lib.check(_lib.load().sf_compact(_lib.ptr(f), f.stride(0), f.stride(1), _lib.dtype_code(f, "f"), M, N,
                                              _lib.ptr(indptr), nnz, _lib.ptr(indices), _lib.ptr(values),
                                              _lib.stream(dev)))
    return indices, values


def dense_to_csr(f, row_nnz=None):
    """CSR of dense features f [M, d_sae]: (indptr int64 [M+1], indices int32 [nnz], values [nnz]),
    each row's nonzeros in column order.

    row_nnz: per-row nonzero counts if already known (fused_encode produces them);
    otherwise counted here. One host sync (reading indptr[-1]) sizes the outputs.
    """
    M, N = f.shape
    _lib.require_gpu(("f", f), ("row_nnz", row_nnz))
    _lib.dtype_code(f, "f")
    if row_nnz is None:
        row_nnz = row_counts(f)
    elif row_nnz.numel() != M:
        raise ValueError(f"row_nnz has {row_nnz.numel()} entries, f has {M} rows")
    indptr = exclusive_scan(row_nnz)
    nnz = int(indptr[-1])
    indices, values = compact(f, indptr, nnz)
    return indptr, indices, values


def _csr_parts(indptr, indices, values):
    if indptr.dtype != torch.int64 or indptr.dim() != 1 or indptr.numel() < 1:
        raise ValueError("indptr must be a 1-D int64 tensor of M+1 offsets")
    if indices.numel() != values.numel():
        raise ValueError(f"indices ({indices.numel()}) and values ({values.numel()}) differ in length")
    indptr = indptr.contiguous()
    indices = indices.reshape(-1)
    if indices.dtype != torch.int32:
        if indices.dtype not in (torch.int64, torch.int16, torch.uint8, torch.int8):
            raise ValueError(f"indices must be an integer tensor, got {indices.dtype}")
        indices = indices.to(torch.int32)
    return indptr, indices.contiguous(), values.reshape(-1).contiguous()


def sparse_decode(indptr, indices, values, W_dec, b_dec=None, *, out_dtype=None, config=None):
    """Reconstruction from CSR features: [M, d_in] rows b_dec + sum of value * W_dec row, with
    fp32 sums (b_dec optional).

    W_dec: [d_sae, d_in] with any strides; row-major is the fast layout, and rows of whole
      128-B lines (d_in a multiple of 64 in 16-bit, of 32 in fp32) take the line-slab kernel,
      whose XCDs each gather one 128-B column slab of W_dec at a time from their L2.
    config: None, or a dict with BLOCK_NNZ and BLOCK_D (num_warps may be present and is
      ignored) that pins the one-wavefront-per-row kernel: BLOCK_D is the d_in slab one
      wavefront covers, rounded up to whole 16-B chunks per lane; BLOCK_NNZ must be positive
      (entries are gathered 64 at a time). Results do not depend on it.
    """
    M = indptr.numel() - 1
    d_sae, D = W_dec.shape
    out = torch.empty(M, D, device=W_dec.device, dtype=out_dtype or W_dec.dtype)
    if M == 0:
        return out
    dev = _lib.require_gpu(("indptr", indptr), ("indices", indices), ("values", values), ("W_dec", W_dec),
                           ("b_dec", b_dec))
    indptr, indices, values = _csr_parts(indptr, indices, values)
    if b_dec is not None:
        if b_dec.numel() != D:
            raise ValueError(f"b_dec must have {D} entries, got {b_dec.numel()}")
        b_dec = b_dec.reshape(D).contiguous()
    cfg = None
    if config is not None:
        try:
            cfg = (ctypes.c_int32 * 2)(int(config["BLOCK_NNZ"]), int(config["BLOCK_D"]))
        except (TypeError, KeyError, ValueError):
            raise ValueError(f"config must be a dict with BLOCK_NNZ and BLOCK_D, got {config!r}") from None
    lib = _lib.load()
    with torch.cuda.device(dev):
        _lib.check(lib.sf_decode(
            _lib.ptr(indptr), _lib.ptr(indices), _lib.ptr(values), _lib.dtype_code(values, "values"), values.numel(),
            _lib.ptr(W_dec), W_dec.stride(0), W_dec.stride(1), _lib.dtype_code(W_dec, "W_dec"), d_sae,
            _lib.ptr(b_dec), _lib.dtype_code(b_dec, "b_dec") if b_dec is not None else 0,
            _lib.ptr(out), out.stride(0), out.stride(1), _lib.dtype_code(out, "out"), M, D, cfg, _lib.stream(dev)))
    return out


def csr_to_dense(indptr, indices, values, d_sae):
    """Inverse of dense_to_csr: [M, d_sae] in the values' dtype (duplicate columns are summed)."""
    M = indptr.numel() - 1
    out = torch.empty(M, d_sae, device=values.device, dtype=values.dtype)
    if M == 0 or d_sae == 0:
        return out
    dev = _lib.require_gpu(("indptr", indptr), ("indices", indices), ("values", values))
    indptr, indices, values = _csr_parts(indptr, indices, values)
    lib = _lib.load()
    code = _lib.dtype_code(values, "values")
    with torch.cuda.device(dev):
        _lib.check(lib.sf_csr_to_dense(_lib.ptr(indptr), 0, _lib.ptr(indices), _lib.ptr(values), code,
                                       values.numel(), M, d_sae, _lib.ptr(out), out.stride(0), code,
                                       _lib.stream(dev)))
    return out


def topk_rows(f, k):
    """Row-wise top-k of f [M, N]: (values [M, k] sorted descending, indices int32 [M, k]).

    The selection of f.topk(k, dim=-1) (ops.py:16) for any 0 <= k <= N; ties are taken
    and ordered by increasing column.
    """
    M, N = f.shape
    if not 0 <= k <= N:
        raise RuntimeError(f"selected index k out of range: k={k}, N={N}")
    values = torch.empty(M, k, device=f.device, dtype=f.dtype)
    indices = torch.empty(M, k, device=f.device, dtype=torch.int32)
    if M == 0 or k == 0:
        return values, indices
    dev = _lib.require_gpu(("f", f))
    lib = _lib.load()
    with torch.cuda.device(dev):
        _lib.check(lib.sf_topk(_lib.ptr(f), f.stride(0), f.stride(1), _lib.dtype_code(f, "f"), M, N, k,
                               _lib.ptr(values), _lib.ptr(indices), _lib.stream(dev)))
    return values, indices


def topk_gather(f, k, n_rows, out_rows, values, indices, *, row_off=0):
    """topk_rows of the live rows i < clamp(n_rows - row_off, 0, M) of f [M, N] (n_rows: an
    int32 count in device memory), row i written into row out_rows[row_off + i] of the given
    values / indices [M_out, k]; no other row of them is touched and nothing is read back."""
    M, N = f.shape
    if not 0 <= k <= N:
        raise RuntimeError(f"selected index k out of range: k={k}, N={N}")
    if values.shape != indices.shape or values.dim() != 2 or values.shape[1] != k or not values.is_contiguous() \
            or not indices.is_contiguous() or indices.dtype != torch.int32 or values.dtype != f.dtype:
        raise ValueError("values / indices must be contiguous [M_out, k] tensors of f's dtype and int32")
    if M == 0 or k == 0:
        return
    dev = _lib.require_gpu(("f", f), ("n_rows", n_rows), ("out_rows", out_rows), ("values", values),
                           ("indices", indices))
    with torch.cuda.device(dev):
        _lib.check(_lib.load().sf_topk_gather(_lib.ptr(f), f.stride(0), f.stride(1), _lib.dtype_code(f, "f"), M, N, k,
                                              _lib.ptr(n_rows), row_off, _lib.ptr(out_rows), values.shape[0],
                                              _lib.ptr(values), _lib.ptr(indices), _lib.stream(dev)))


def overflow_rows(cand_cnt, cap):
    """(rows int32 [M], n int32 [1]), both on the device: rows[:n] are the rows with
    cand_cnt > cap in increasing order. Nothing is read back to the host."""
    M = cand_cnt.numel()
    dev = _lib.require_gpu(("cand_cnt", cand_cnt))
    rows = torch.empty(M, dtype=torch.int32, device=cand_cnt.device)
    n = torch.empty(1, dtype=torch.int32, device=cand_cnt.device)
    with torch.cuda.device(dev):
        _lib.check(_lib.load().sf_overflow_rows(_lib.ptr(cand_cnt.contiguous()), M, cap, _lib.ptr(rows), _lib.ptr(n),
                                                _lib.stream(dev)))
    return rows, n


def fixed_width_to_dense(indices, values, d_sae):
    """Dense [M, d_sae] from fixed-width rows (indices/values [M, k]), the TopK scatter
    `zeros.scatter_(-1, indices, values)` (ops.py:21-25)."""
    M, k = indices.shape
    out = torch.empty(M, d_sae, device=values.device, dtype=values.dtype)
    if M == 0 or d_sae == 0:
        return out
    dev = _lib.require_gpu(("indices", indices), ("values", values))
    indices = indices.to(torch.int32).contiguous()
    values = values.contiguous()
    lib = _lib.load()
    code = _lib.dtype_code(values, "values")
    with torch.cuda.device(dev):
        _lib.check(lib.sf_csr_to_dense(None, k, _lib.ptr(indices), _lib.ptr(values), code, values.numel(), M, d_sae,
                                       _lib.ptr(out), out.stride(0), code, _lib.stream(dev)))
    return out


def rows_to_csr(cand_cnt, cand_idx, cand_val, indptr, nnz):
    """Row candidates (encode_rows) -> canonical CSR (indices int32 [nnz], values [nnz]), rows
    sorted by column; indptr = exclusive_scan(cand_cnt). Rows whose list overflowed (cand_cnt >
    cap) are skipped: their segments of the returned arrays are left unset for the caller to
    fill (as ops._fill_overflowed_rows does)."""
    M, cap = cand_idx.shape
    dev = _lib.require_gpu(("cand_cnt", cand_cnt), ("cand_idx", cand_idx), ("cand_val", cand_val),
                           ("indptr", indptr))
    indices = torch.empty(nnz, dtype=torch.int32, device=cand_idx.device)
    values = torch.empty(nnz, dtype=cand_val.dtype, device=cand_idx.device)
    if M == 0 or nnz == 0:
        return indices, values
    lib = _lib.load()
    with torch.cuda.device(dev):
        _lib.check(lib.sf_rows_to_csr(_lib.ptr(cand_cnt), _lib.ptr(cand_idx), _lib.ptr(cand_val),
                                      _lib.dtype_code(cand_val, "cand_val"), cap, M, _lib.ptr(indptr), nnz,
                                      _lib.ptr(indices), _lib.ptr(values), _lib.stream(dev)))
    return indices, values


def rows_topk(cand_cnt, cand_idx, cand_val, k, n_features):
    """Row-wise top-k of row candidates: (values [M, k] sorted descending, indices int32 [M, k]),
    equal values by increasing column, as topk_rows on the dense rows."""
    M, cap = cand_idx.shape
    if k > n_features:
        raise RuntimeError(f"selected index k out of range (k={k}, N={n_features})")
    dev = _lib.require_gpu(("cand_cnt", cand_cnt), ("cand_idx", cand_idx), ("cand_val", cand_val))
    values = torch.empty(M, k, device=cand_idx.device, dtype=cand_val.dtype)
    indices = torch.empty(M, k, device=cand_idx.device, dtype=torch.int32)
    if M == 0 or k == 0:
        return values, indices
    lib = _lib.load()
    with torch.cuda.device(dev):
        _lib.check(lib.sf_rows_topk(_lib.ptr(cand_cnt), _lib.ptr(cand_idx), _lib.ptr(cand_val),
                                    _lib.dtype_code(cand_val, "cand_val"), cap, M, n_features, k,
                                    _lib.ptr(values), _lib.ptr(indices), _lib.stream(dev)))
    return values, indices
