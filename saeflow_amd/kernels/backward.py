"""Backward of the sparse SAE path on the gfx950 kernels (C ABI, include/saeflow_hip.h).

The reference lists backward kernels for training SAEs on sparse features on its roadmap
(saeflow README.md:244). The forward they differentiate is the reference's
(reference.py:36-52, with the CSR of ops.encode_sparse, ops.py:29-39):

    x' = cast_W(x - b_dec),  pre = x' W_enc + b_enc,  f = act(pre),  x_hat = f W_dec + b_dec

act is relu, jumprelu or the top-k of relu; on the CSR's nonzeros act'(pre) = 1 and
elsewhere 0, so every gradient is a sum over the nonzeros.
"""

import ctypes
from types import SimpleNamespace

import torch

from .. import _lib


def _rows(t, dtype):
    """t as `dtype` with unit column stride (a copy only when needed)."""
    if t.dtype != dtype:
        t = t.to(dtype)
    return t if t.stride(-1) == 1 else t.contiguous()


def csr_transpose(indptr, indices, n_cols):
    """CSR [M, n_cols] -> (colptr int64 [n_cols+1], rows int32 [nnz], positions int32 [nnz]):
    per column, its entries' rows in increasing order and their positions in the CSR arrays.
    Deterministic. Entries whose index is outside [0, n_cols) are left out."""
    M = indptr.numel() - 1
    nnz = indices.numel()
    dev = _lib.require_gpu(("indptr", indptr), ("indices", indices))
    lib = _lib.load()
    colptr = torch.empty(n_cols + 1, dtype=torch.int64, device=dev)
    rows = torch.empty(nnz, dtype=torch.int32, device=dev)
    pos = torch.empty(nnz, dtype=torch.int32, device=dev)
    nbytes = ctypes.c_int64()
    _lib.check(lib.sf_csr_transpose_workspace_size(M, n_cols, nnz, ctypes.byref(nbytes)))
    ws = torch.empty(nbytes.value, dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        _lib.check(lib.sf_csr_transpose(_lib.ptr(indptr), _lib.ptr(indices), M, n_cols, nnz, _lib.ptr(colptr),
                                        _lib.ptr(rows), _lib.ptr(pos), _lib.ptr(ws), nbytes.value,
                                        _lib.stream(dev)))
    return colptr, rows, pos


def sparse_backward(x, W_enc, b_enc, W_dec, b_dec, csr, grad_x_hat=None, grad_values=None, *, need_grad_x=True):
    """Gradients of a loss L through the forward above, from g_xhat = dL/dx_hat [M, d_in] and
    optionally dL/df on the CSR values (grad_values [nnz], e.g. from a sparsity penalty).

    csr = (indptr, indices, values) as encode_sparse returned it for x. Returns a namespace
    with W_enc [d_in, d_sae], b_enc, W_dec [d_sae, d_in], b_dec (each in its parameter's
    dtype), x (x's dtype; None unless need_grad_x) and pre (fp32 dL/dpre on the CSR entries).
    fp32 accumulation throughout, in a fixed order (repeated calls give identical bits). No
    threshold gradient: jumprelu's is zero almost everywhere. Nothing waits for the GPU.
    """
    indptr, indices, values = csr
    M, D = x.shape
    if W_enc.shape[0] != D or W_dec.shape != (W_enc.shape[1], D):
        raise ValueError(f"shape mismatch: x {tuple(x.shape)}, W_enc {tuple(W_enc.shape)}, W_dec {tuple(W_dec.shape)}")
    N = W_enc.shape[1]
    if W_enc.dtype != W_dec.dtype:
        raise ValueError(f"W_enc ({W_enc.dtype}) and W_dec ({W_dec.dtype}) must share a dtype")
    dev = _lib.require_gpu(("x", x), ("W_enc", W_enc), ("b_enc", b_enc), ("W_dec", W_dec), ("b_dec", b_dec),
                           ("indptr", indptr), ("indices", indices), ("values", values),
                           ("grad_x_hat", grad_x_hat), ("grad_values", grad_values))
    if indptr.numel() != M + 1:
        raise ValueError(f"indptr has {indptr.numel()} entries for {M} rows")
    dt = W_dec.dtype
    code = _lib.dtype_code(W_dec, "W_dec")
    nnz = indices.numel()
    lib = _lib.load()
    with torch.cuda.device(dev):
        s = _lib.stream(dev)
        g = torch.zeros(M, D, dtype=dt, device=dev) if grad_x_hat is None else _rows(grad_x_hat, dt)
        Wd = _rows(W_dec, dt)
        gv = None if grad_values is None else grad_values.reshape(-1)
        if gv is not None and gv.numel() != nnz:
            raise ValueError(f"grad_values has {gv.numel()} entries for nnz={nnz}")
        # per-feature sums over the CSC
        colptr, rows, pos = csr_transpose(indptr, indices, N)
        xs = torch.empty(M, D, dtype=dt, device=dev)
        _lib.check(lib.sf_shifted_input(_lib.ptr(x), x.stride(0), x.stride(1), _lib.dtype_code(x, "x"),
                                        _lib.ptr(b_dec), _lib.dtype_code(b_dec, "b_dec"), M, D, code, _lib.ptr(xs), s))
        plan_i64 = torch.empty(3 * (N + 1), dtype=torch.int64, device=dev)
        max_items, max_slots, work_floats = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
        _lib.check(lib.sf_backward_bounds(N, nnz, D, code, ctypes.byref(max_items), ctypes.byref(max_slots),
                                          ctypes.byref(work_floats)))
        item_col = torch.empty(max_items.value, dtype=torch.int32, device=dev)
        multi_col = torch.empty(N, dtype=torch.int32, device=dev)
        slot_item = torch.empty(max_slots.value, dtype=torch.int32, device=dev)
        _lib.check(lib.sf_backward_plan(_lib.ptr(colptr), N, nnz, _lib.ptr(plan_i64), _lib.ptr(item_col),
                                        _lib.ptr(multi_col), _lib.ptr(slot_item), s))
        g_pre = torch.empty(nnz, dtype=torch.float32, device=dev)  # dL/dpre on the nonzeros
        d_wdec = torch.empty(N, D, dtype=dt, device=dev)
        d_wenc = torch.empty(D, N, dtype=dt, device=dev)
        d_benc = torch.empty(N, dtype=torch.float32, device=dev)
        partials = torch.empty(max_slots.value * (2 * D + 1), dtype=torch.float32, device=dev)
        work = torch.empty(work_floats.value, dtype=torch.float32, device=dev)
        # the grid is sized by the bound of the work-item count (surplus waves return at once), so
        # nothing here waits for the GPU
        _lib.check(lib.sf_backward_columns(_lib.ptr(colptr), _lib.ptr(rows), _lib.ptr(pos), _lib.ptr(plan_i64),
                                           _lib.ptr(item_col), _lib.ptr(multi_col), _lib.ptr(slot_item),
                                           max_items.value, max_slots.value,
                                           _lib.ptr(values), _lib.dtype_code(values, "values"), _lib.ptr(gv),
                                           0 if gv is None else _lib.dtype_code(gv, "grad_values"), _lib.ptr(Wd),
                                           Wd.stride(0), _lib.ptr(xs), D, _lib.ptr(g), g.stride(0), code, N, M, D,
                                           nnz, _lib.ptr(g_pre), _lib.ptr(d_wdec), _lib.ptr(d_wenc),
                                           _lib.ptr(d_benc), _lib.ptr(partials), _lib.ptr(work), work.numel(), s))
        del partials, xs, work
        # db_dec = sum_m g_xhat[m] - sum_m dx'[m], and sum_m dx'[m] = W_enc db_enc
        d_bdec = torch.empty(D, dtype=torch.float32, device=dev)
        ws = torch.empty(min(256, max(M, 1)) * D, dtype=torch.float32, device=dev)
        _lib.check(lib.sf_column_sums(_lib.ptr(g), M, D, g.stride(0), code, 1.0, 0, _lib.ptr(d_bdec), _lib.ptr(ws),
                                      ws.numel(), s))
        mv_ws = torch.empty(D * min(256, max(N, 1)), dtype=torch.float32, device=dev)
        _lib.check(lib.sf_matvec(_lib.ptr(W_enc), D, N, W_enc.stride(0), W_enc.stride(1), code, _lib.ptr(d_benc),
                                 -1.0, 1, _lib.ptr(d_bdec), _lib.ptr(mv_ws), mv_ws.numel(), s))
        dxs = None
        if need_grad_x:  # dx' = g_pre W_enc^T: the forward decode over the rows of W_enc^T
            if W_enc.stride(0) == 1:  # W_enc is the transpose of a row-major [d_sae, d_in]
                W_encT = W_enc.t()
            else:
                W_encT = torch.empty(N, D, dtype=dt, device=dev)
                We = _rows(W_enc, dt)
                _lib.check(lib.sf_transpose(_lib.ptr(We), D, N, We.stride(0), code, None, _lib.ptr(W_encT), s))
            dxs = torch.empty(M, D, dtype=torch.float32, device=dev)
            _lib.check(lib.sf_decode(_lib.ptr(indptr), _lib.ptr(indices), _lib.ptr(g_pre), _lib.DTYPE[torch.float32],
                                     nnz, _lib.ptr(W_encT), W_encT.stride(0), W_encT.stride(1), code, N, None, 0,
                                     _lib.ptr(dxs), D, 1, _lib.DTYPE[torch.float32], M, D, None, s))
    return SimpleNamespace(W_enc=d_wenc.to(W_enc.dtype), b_enc=d_benc.to(b_enc.dtype), W_dec=d_wdec,
                           b_dec=d_bdec.to(b_dec.dtype), x=None if dxs is None else dxs.to(x.dtype), pre=g_pre)
