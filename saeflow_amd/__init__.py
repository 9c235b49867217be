"""saeflow_amd: the saeflow SAE hot path (fused encode -> dense->CSR -> sparse decode)
as hand-written HIP kernels for MI355X (gfx950), behind saeflow's public API
(reference saeflow/__init__.py:3-7)."""

from .ops import decode_sparse, encode, encode_sparse, forward
from .sae import SAE
from .training import forward_train

__version__ = "0.1.0"
__all__ = ["SAE", "decode_sparse", "encode", "encode_sparse", "forward", "forward_train"]
