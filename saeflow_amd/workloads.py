"""Synthetic SAE workloads of the benchmark configurations (seeded, reproducible).

Five configurations, by name:
  C1  relu      fp32  d_in=768   d_sae=24576    T=2048   b_enc=-2.8 (L0 about 63)
  C2  jumprelu  bf16  d_in=2304  d_sae=16384    T=16384  L0=64
  C3  jumprelu  bf16  d_in=2304  d_sae=65536    T=16384  L0=64   (headline)
  C4  topk      fp16  d_in=4096  d_sae=131072   T=8192   k=32
  C5  jumprelu  bf16  d_in=2304  d_sae=1048576  T=4096   L0=128

Recipe: W_enc ~ N(0, 1/d_in); W_dec = W_enc^T with unit-norm rows; b_dec ~ N(0, 0.1^2);
x = b_dec + N(0, 1), so every pre-activation is about N(0, 1). JumpReLU configs draw a
per-feature firing probability p_i ~ LogNormal(0, 1.5), rescaled to sum to L0 and clipped
at 0.5 (repeated until the sum is within 0.5 of L0), set theta_i = Phi^-1(1 - p_i) and
b_enc = 0, so E[L0] = sum p_i. ReLU and TopK configs use b_enc = -2.8.

Everything is drawn in fp32 from one torch.Generator on the given device in a fixed order
and then rounded to the config dtype: the same seed and device give identical tensors. The
CPU and GPU generators draw different streams, so a CPU-made workload differs from a
GPU-made one of the same seed (tests that compare against the CPU oracle copy the GPU
tensors to the CPU, or build on the CPU and copy to the GPU).
"""

import math
from types import SimpleNamespace

import torch

CONFIGS = {
    "C1": dict(activation="relu", dtype=torch.float32, d_in=768, d_sae=24576, T=2048, l0=64, b_enc=-2.8),
    "C2": dict(activation="jumprelu", dtype=torch.bfloat16, d_in=2304, d_sae=16384, T=16384, l0=64),
    "C3": dict(activation="jumprelu", dtype=torch.bfloat16, d_in=2304, d_sae=65536, T=16384, l0=64),
    "C4": dict(activation="topk", dtype=torch.float16, d_in=4096, d_sae=131072, T=8192, k=32, b_enc=-2.8),
    "C5": dict(activation="jumprelu", dtype=torch.bfloat16, d_in=2304, d_sae=1048576, T=4096, l0=128),
}
HEADLINE = "C3"


def firing_probabilities(d_sae, l0, g, device):
    """p_i ~ LogNormal(0, 1.5), rescaled to sum l0, clipped at 0.5, iterated; returns (p, sum)."""
    p = torch.exp(1.5 * torch.randn(d_sae, generator=g, device=device, dtype=torch.float64))
    for _ in range(200):
        p = (p * (l0 / p.sum())).clamp(max=0.5)
        if abs(float(p.sum()) - l0) <= 0.5:
            break
    return p, float(p.sum())


def make(name, *, seed=0, device="cpu", T=None, d_sae=None, d_in=None, dtype=None):
    """SAE-like namespace (W_enc, b_enc, W_dec, b_dec, threshold, activation, k) plus x and
    metadata for config `name`; T / d_sae / d_in / dtype override the config for scaled-down
    parity cases."""
    cfg = dict(CONFIGS[name])
    T = T or cfg["T"]
    d_sae = d_sae or cfg["d_sae"]
    d_in = d_in or cfg["d_in"]
    dtype = dtype or cfg["dtype"]
    g = torch.Generator(device=device).manual_seed(seed)
    W_enc = torch.randn(d_in, d_sae, generator=g, device=device) / math.sqrt(d_in)
    b_dec = torch.randn(d_in, generator=g, device=device) * 0.1
    x = b_dec + torch.randn(T, d_in, generator=g, device=device)
    threshold, l0_expected = None, None
    if cfg["activation"] == "jumprelu":
        l0 = cfg["l0"] * d_sae / cfg["d_sae"] if d_sae != cfg["d_sae"] else cfg["l0"]
        p, l0_expected = firing_probabilities(d_sae, l0, g, device)
        threshold = torch.special.ndtri(1.0 - p).float()
        b_enc = torch.zeros(d_sae, device=device)
    else:
        b_enc = torch.full((d_sae,), cfg["b_enc"], device=device)
    W_dec = W_enc.T / W_enc.T.norm(dim=1, keepdim=True)
    sae = SimpleNamespace(
        W_enc=W_enc.to(dtype),
        W_dec=W_dec.contiguous().to(dtype),
        b_enc=b_enc.to(dtype),
        b_dec=b_dec.to(dtype),
        threshold=None if threshold is None else threshold.to(dtype),
        activation=cfg["activation"],
        k=cfg.get("k"),
        d_in=d_in,
        d_sae=d_sae,
    )
    del W_enc, W_dec
    meta = dict(name=name, T=T, d_in=d_in, d_sae=d_sae, dtype=dtype, activation=cfg["activation"],
                l0_target=cfg.get("l0"), l0_expected=l0_expected, k=cfg.get("k"), seed=seed)
    return sae, x.to(dtype), meta


def encode_flops(T, d_in, d_sae):
    """2*T*d_in*d_sae (reference bench/bench_encode.py:72)."""
    return 2 * T * d_in * d_sae


def compaction_bytes(T, d_sae, nnz, esize):
    """T*d_sae*e + nnz*(4+e) + (T+1)*8 (reference bench/bench_decode.py:89, M*l0 -> nnz)."""
    return T * d_sae * esize + nnz * (4 + esize) + (T + 1) * 8


def decode_bytes(T, d_in, nnz, esize):
    """nnz*(d_in*e + 4 + e) + T*d_in*e + (T+1)*8 (reference bench/bench_decode.py:57, M*l0 -> nnz)."""
    return nnz * (d_in * esize + 4 + esize) + T * d_in * esize + (T + 1) * 8


def backward_bytes(T, d_in, d_sae, nnz, esize, grad_x=False):
    """Algorithmic bytes of sparse_backward (no reference formula: the reference has no
    backward). Requested, as the decode formula counts them, with nslab = ceil(d_in*e / 1024)
    slabs of d_in per feature:
      dW_dec and dots   nnz*d_in*e (gathered g_xhat rows) + nnz*(4 + 4 + e) (CSC row and
                        position, f) + 2*d_sae*d_in*e (W_dec rows in, dW_dec out) + nnz*nslab*4
      dL/dpre           nnz*(nslab*4 + 4 + e + 4 + 4) (slab dots, position, f in; g_pre and its
                        CSC-order copy out)
      dW_enc, db_enc    nnz*d_in*e (gathered x' rows) + nnz*(4 + 4) + d_sae*d_in*e (out, written
                        in its [d_in, d_sae] layout)
      x'                2*T*d_in*e
      db_dec            T*d_in*e (column sums of g_xhat) + d_sae*d_in*e (W_enc db_enc)
      dx' (grad_x)      decode_bytes over W_enc^T plus its transpose 2*d_sae*d_in*e."""
    row = d_in * esize
    nslab = -(-row // 1024)
    b = nnz * row + nnz * (8 + esize) + 2 * d_sae * row + nnz * nslab * 4
    b += nnz * (nslab * 4 + 12 + esize)
    b += nnz * row + nnz * 8 + d_sae * row
    b += 2 * T * row
    b += T * row + d_sae * row
    if grad_x:
        b += decode_bytes(T, d_in, nnz, esize) + 2 * d_sae * row
    return b
