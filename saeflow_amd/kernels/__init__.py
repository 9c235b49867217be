"""gfx950 kernel wrappers (reference saeflow/kernels/__init__.py:6-9)."""

from .decode import (compact, csr_to_dense, dense_to_csr, exclusive_scan, fixed_width_to_dense, row_counts,
                     sparse_decode, topk_rows)
from .encode import best_config, encode_pre, fused_encode

__all__ = ["best_config", "compact", "csr_to_dense", "dense_to_csr", "encode_pre", "exclusive_scan",
           "fixed_width_to_dense", "fused_encode", "row_counts", "sparse_decode", "topk_rows"]
