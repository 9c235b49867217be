"""Writes the golden fixtures of tests/golden/*.npz from the brute-force pins.

    python tests/golden/make_golden.py

Inputs are small seeded tensors (rounded to bf16 where the case says so, and stored as
the float32 values of those rounded numbers); expected outputs come from oracle.brute, the
element-by-element float64 statement of the reference formulas (reference.py:36-49,
decode.py:28-74, ops.py:16). The reference's own tests commit no vectors, so these are
the fixed points that pin the vectorised oracle and the GPU kernels.
"""

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import brute  # noqa: E402


def lst(a):
    return np.asarray(a, dtype=np.float64).tolist()


def encode_case(name, M, K, N, activation, seed, round_bf16=False, k=None):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    W = torch.randn(K, N, generator=g) / K ** 0.5
    b_enc = torch.randn(N, generator=g) * 0.1
    b_dec = torch.randn(K, generator=g) * 0.1
    thr = torch.rand(N, generator=g) * 0.5
    if round_bf16:
        x, W, b_enc, b_dec, thr = (t.to(torch.bfloat16).float() for t in (x, W, b_enc, b_dec, thr))
    pre, out = brute.encode(lst(x), lst(W), lst(b_enc), lst(b_dec), lst(thr), activation, k)
    np.savez(HERE / f"{name}.npz", x=x.numpy(), W_enc=W.numpy(), b_enc=b_enc.numpy(), b_dec=b_dec.numpy(),
             threshold=thr.numpy(), pre=np.array(pre), out=np.array(out), activation=np.array(activation),
             k=np.array(k or 0), bf16=np.array(round_bf16))


def csr_case():
    g = torch.Generator().manual_seed(7)
    f = torch.relu(torch.randn(6, 23, generator=g) - 0.8)
    f[0] = 0.0            # empty row
    f[3, 5] = -0.0        # negative zero is zero
    f[4] = 0.0
    f[4, 22] = 2.5        # last column only
    f[5, 0] = -1.25       # negative nonzero at column 0
    indptr, indices, values = brute.dense_to_csr(lst(f))
    np.savez(HERE / "csr.npz", f=f.numpy(), indptr=np.array(indptr, np.int64), indices=np.array(indices, np.int32),
             values=np.array(values, np.float32))


def decode_case():
    g = torch.Generator().manual_seed(11)
    d_sae, D, M = 9, 6, 4
    W = torch.randn(d_sae, D, generator=g)
    b = torch.randn(D, generator=g) * 0.1
    indptr = [0, 3, 3, 7, 8]  # row 1 empty
    indices = [0, 4, 8, 1, 2, 4, 8, 5]
    values = torch.randn(len(indices), generator=g).tolist()
    out = brute.sparse_decode(indptr, indices, values, lst(W), lst(b))
    np.savez(HERE / "decode.npz", W_dec=W.numpy(), b_dec=b.numpy(), indptr=np.array(indptr, np.int64),
             indices=np.array(indices, np.int32), values=np.array(values, np.float32), out=np.array(out),
             M=np.array(M))


def topk_case():
    f = np.array([[0.5, 2.0, 2.0, -1.0, 3.0, 0.0, 2.0, 0.25],
                  [0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 1.0],
                  [-3.0, -1.0, -2.0, -1.0, -5.0, -1.0, -4.0, -0.5]], dtype=np.float32)
    vals, cols = brute.topk(f.tolist(), 3)
    np.savez(HERE / "topk.npz", f=f, k=np.array(3), values=np.array(vals), cols=np.array(cols, np.int32))


if __name__ == "__main__":
    encode_case("encode_relu", 3, 5, 7, "relu", seed=1)
    encode_case("encode_jumprelu", 4, 6, 5, "jumprelu", seed=2)
    encode_case("encode_topk", 3, 4, 9, "topk", seed=3, k=3)
    encode_case("encode_relu_bf16", 5, 16, 24, "relu", seed=4, round_bf16=True)
    csr_case()
    decode_case()
    topk_case()
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))
