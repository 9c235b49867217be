"""The SAE parameter container of saeflow's public API (reference saeflow/reference.py:9-34).

Same constructor, parameter names, shapes and initialisation as the reference module;
its methods run on this package's gfx950 kernels, so `sae(x)` and `sae.encode(x)` are the
GPU path, not a plain-PyTorch re-computation.
"""

import torch
from torch import nn

ACTIVATIONS = ("relu", "jumprelu", "topk")


class SAE(nn.Module):
    """Sparse autoencoder parameters: features f = act((x - b_dec) W_enc + b_enc) and the
    reconstruction x_hat = f W_dec + b_dec.

    Activations: "relu"; "jumprelu", which also zeroes features at or below their own
    `threshold`; "topk", which keeps each token's `k` largest ReLU features. The tensors carry
    SAELens's names and layouts (W_enc is [d_in, d_sae], W_dec is [d_sae, d_in]).
    """

    def __init__(self, d_in, d_sae, activation="relu", k=None, device=None, dtype=torch.float32):
        super().__init__()
        if activation not in ACTIVATIONS:
            raise ValueError(f"activation must be one of {ACTIVATIONS}, got {activation!r}")
        if activation == "topk" and not k:
            raise ValueError("topk activation needs k")
        self.d_in, self.d_sae, self.activation, self.k = d_in, d_sae, activation, k

        W_dec = torch.randn(d_sae, d_in, device=device)
        W_dec /= W_dec.norm(dim=1, keepdim=True)
        self.W_dec = nn.Parameter(W_dec.to(dtype))
        self.W_enc = nn.Parameter(W_dec.T.contiguous().to(dtype))
        self.b_enc = nn.Parameter(torch.zeros(d_sae, device=device, dtype=dtype))
        self.b_dec = nn.Parameter(torch.zeros(d_in, device=device, dtype=dtype))
        self.threshold = (
            nn.Parameter(torch.zeros(d_sae, device=device, dtype=dtype)) if activation == "jumprelu" else None
        )
        self.requires_grad_(False)

    def encode_pre(self, x):
        from .kernels import encode_pre

        return encode_pre(x, self.W_enc, self.b_enc, self.b_dec)

    def encode(self, x):
        from .ops import encode

        return encode(self, x)

    def decode(self, f):
        """Dense features [M, d_sae] -> [M, d_in], through the CSR path (compaction + gather)."""
        from .kernels import dense_to_csr
        from .ops import decode_sparse

        return decode_sparse(self, dense_to_csr(f))

    def forward(self, x):
        from .ops import forward

        return forward(self, x)
