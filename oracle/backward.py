"""Gradients of the SAE forward on the CPU — test infrastructure (see oracle/__init__.py).

Differentiates the forward of saeflow/reference.py:36-52 (pre = (x - b_dec) @ W_enc + b_enc,
f = act(pre), x_hat = f @ W_dec + b_dec) with torch autograd in float64, for the loss
L = sum(x_hat * G) + sum(f * H): G plays dL/dx_hat and H dL/df. The activation is taken as
`pre * active`, where `active` is the given set of nonzeros (the CSR the GPU encode produced):
on that set act'(pre) = 1 and off it 0 for relu, jumprelu and the top-k of relu, so this is
their derivative without re-deciding threshold ties. The reference has no backward kernels
(they are on its roadmap, README.md:244); this is the mathematics they must reproduce.

Pinned in tests/test_oracle.py by central finite differences of the same loss and by the
closed forms dW_dec = f^T G and db_enc = colsum((G W_dec^T + H) * active).
"""

import torch


def grads(x, W_enc, b_enc, W_dec, b_dec, active, G, H=None):
    """dL/d{x, W_enc, b_enc, W_dec, b_dec} (float64) and the features f, for
    L = sum(x_hat * G) + sum(f * H), f = ((x - b_dec) @ W_enc + b_enc) * active."""
    leaves = [t.detach().to("cpu", torch.float64).requires_grad_(True) for t in (x, W_enc, b_enc, W_dec, b_dec)]
    xx, We, be, Wd, bd = leaves
    f = ((xx - bd) @ We + be) * active.to(torch.float64)
    x_hat = f @ Wd + bd
    loss = (x_hat * G.to(torch.float64)).sum()
    if H is not None:
        loss = loss + (f * H.to(torch.float64)).sum()
    loss.backward()
    return {"x": xx.grad, "W_enc": We.grad, "b_enc": be.grad, "W_dec": Wd.grad, "b_dec": bd.grad,
            "f": f.detach()}
