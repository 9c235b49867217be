"""Plain-PyTorch SAE math on the CPU — test infrastructure (see oracle/__init__.py).

Restates saeflow/reference.py:36-52 (SAE.encode_pre / encode / decode / forward) and the
SAE-level semantics of saeflow/ops.py:12-49, as functions of explicit parameters. Inputs
are upcast to the compute dtype (float32 by default, float64 on request) from the same
rounded low-precision tensors the GPU gets, as the reference tests do
(tests/test_kernels.py:33-37).
"""

import torch


def _c(t, dtype):
    return None if t is None else t.detach().to("cpu", dtype)


def encode_pre(x, W_enc, b_enc, b_dec, dtype=torch.float32):
    """(x - b_dec) @ W_enc + b_enc  (reference.py:36-37)."""
    return (_c(x, dtype) - _c(b_dec, dtype)) @ _c(W_enc, dtype) + _c(b_enc, dtype)


def activate(pre, activation, threshold=None, k=None):
    """relu / jumprelu / topk of a pre-activation (reference.py:39-46)."""
    if activation == "relu":
        return torch.relu(pre)
    if activation == "jumprelu":
        return torch.relu(pre) * (pre > _c(threshold, pre.dtype))
    if activation == "topk":
        top = pre.topk(k, dim=-1)
        return torch.zeros_like(pre).scatter_(-1, top.indices, torch.relu(top.values))
    raise ValueError(f"unknown activation {activation!r}")


def encode(x, W_enc, b_enc, b_dec, threshold=None, activation="relu", k=None, dtype=torch.float32):
    """Dense features (reference.py:39-46)."""
    return activate(encode_pre(x, W_enc, b_enc, b_dec, dtype), activation, threshold, k)


def decode(f, W_dec, b_dec, dtype=torch.float32):
    """f @ W_dec + b_dec  (reference.py:48-49)."""
    return _c(f, dtype) @ _c(W_dec, dtype) + _c(b_dec, dtype)


def forward(x, W_enc, b_enc, b_dec, W_dec, threshold=None, activation="relu", k=None, dtype=torch.float32):
    """decode(encode(x))  (reference.py:51-52; ops.forward, ops.py:47-49)."""
    return decode(encode(x, W_enc, b_enc, b_dec, threshold, activation, k, dtype), W_dec, b_dec, dtype)


def ops_topk(x, W_enc, b_enc, b_dec, k, dtype=torch.float32):
    """ops._topk (ops.py:12-16): ReLU encode first, then the row top-k (values, indices)."""
    f = torch.relu(encode_pre(x, W_enc, b_enc, b_dec, dtype))
    return f.topk(k, dim=-1)


def sae_params(sae):
    """The attributes ops.py reads from an SAE-like object (ops.py:1-2), as a dict."""
    return dict(W_enc=sae.W_enc, b_enc=sae.b_enc, b_dec=sae.b_dec, W_dec=sae.W_dec,
                threshold=getattr(sae, "threshold", None), activation=sae.activation, k=getattr(sae, "k", None))
