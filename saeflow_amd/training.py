"""Training through the sparse path: the forward of saeflow_amd.forward (encode_sparse then
decode_sparse, ops.py:29-49 in the reference) as a torch.autograd.Function whose backward runs
the gfx950 backward kernels (kernels/backward.py). The reference has these on its roadmap
(saeflow README.md:244); the dense [tokens, d_sae] features exist in neither direction.

    x_hat, (indptr, indices, values) = forward_train(sae, x)
    loss = (x_hat - x).pow(2).sum(-1).mean() + lam * values.float().abs().sum() / len(x)
    loss.backward()      # fills sae.W_enc.grad, b_enc.grad, W_dec.grad, b_dec.grad (and x.grad)

values is differentiable too, so a sparsity penalty on the feature activations (optionally
weighted by W_dec row norms gathered with `indices`) flows back through the encoder.
"""

from types import SimpleNamespace

import torch

from . import ops
from .kernels.backward import sparse_backward


class SparseSAEFunction(torch.autograd.Function):
    """(x, W_enc, b_enc, W_dec, b_dec, threshold, activation, k) -> (x_hat, indptr, indices, values).

    indptr and indices are not differentiable. The threshold gets no gradient (jumprelu's is
    zero almost everywhere; training it needs a pseudo-derivative, which is a modelling choice
    outside the path)."""

    @staticmethod
    def forward(ctx, x, W_enc, b_enc, W_dec, b_dec, threshold, activation, k):
        sae = SimpleNamespace(W_enc=W_enc, b_enc=b_enc, W_dec=W_dec, b_dec=b_dec, threshold=threshold,
                              activation=activation, k=k)
        indptr, indices, values = ops.encode_sparse(sae, x)
        x_hat = ops.decode_sparse(sae, (indptr, indices, values))
        ctx.save_for_backward(x, W_enc, b_enc, W_dec, b_dec, indptr, indices, values)
        ctx.mark_non_differentiable(indptr, indices)
        return x_hat, indptr, indices, values

    @staticmethod
    def backward(ctx, g_xhat, _g_indptr, _g_indices, g_values):
        x, W_enc, b_enc, W_dec, b_dec, indptr, indices, values = ctx.saved_tensors
        need = ctx.needs_input_grad
        if not any(need[:5]):
            return (None,) * 8
        gr = sparse_backward(x, W_enc, b_enc, W_dec, b_dec, (indptr, indices, values), g_xhat, g_values,
                             need_grad_x=need[0])
        return (gr.x if need[0] else None, gr.W_enc if need[1] else None, gr.b_enc if need[2] else None,
                gr.W_dec if need[3] else None, gr.b_dec if need[4] else None, None, None, None)


def forward_train(sae, x):
    """x_hat and the CSR features (indptr, indices, values) of `sae` on x, differentiable with
    respect to x, W_enc, b_enc, W_dec and b_dec (and through `values`)."""
    x_hat, indptr, indices, values = SparseSAEFunction.apply(x, sae.W_enc, sae.b_enc, sae.W_dec, sae.b_dec,
                                                             sae.threshold, sae.activation, sae.k)
    return x_hat, (indptr, indices, values)
