"""gfx950 kernel wrappers (reference saeflow/kernels/__init__.py:6-9)."""

from .decode import (compact, csr_to_dense, dense_to_csr, exclusive_scan, fixed_width_to_dense, overflow_rows,
                     row_counts, rows_to_csr, rows_topk, sparse_decode, topk_gather, topk_rows)
from .backward import csr_transpose, sparse_backward
from .encode import best_config, encode_gather, encode_pre, encode_rows, fused_encode

__all__ = ["best_config", "compact", "csr_to_dense", "csr_transpose", "dense_to_csr", "encode_gather", "encode_pre",
           "encode_rows", "exclusive_scan", "fixed_width_to_dense", "fused_encode", "overflow_rows", "row_counts",
           "rows_to_csr", "rows_topk", "sparse_backward", "sparse_decode", "topk_gather", "topk_rows"]
