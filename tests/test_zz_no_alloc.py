"""GPU: sf_encode_noalloc, the encode whose x' workspace is the library's own device array
(nothing is allocated), against sf_encode with a caller workspace, through the C ABI:
bit-identical features and row counts on two calls in a row, the second with fewer tokens
(the array still holds the first call's x'), token counts beyond one array's worth (encoded
in chunks of whole 256-row blocks), and a d_in too large for one block refused before any
launch."""

import ctypes

import pytest
import torch

from saeflow_amd import _lib, workloads
from saeflow_amd.kernels import fused_encode

pytestmark = pytest.mark.gpu


def encode_noalloc(x, W, b_enc, b_dec, thr, act, out, row_nnz):
    lib = _lib.load()
    M, K = x.shape
    N = W.shape[1]
    dev = x.device
    with torch.cuda.device(dev):
        return lib.sf_encode_noalloc(
            _lib.ptr(x), x.stride(0), x.stride(1), _lib.dtype_code(x, "x"),
            _lib.ptr(W), W.stride(0), W.stride(1), _lib.dtype_code(W, "W_enc"),
            _lib.ptr(b_enc), _lib.dtype_code(b_enc, "b_enc"), _lib.ptr(b_dec), _lib.dtype_code(b_dec, "b_dec"),
            _lib.ptr(thr), _lib.dtype_code(thr, "threshold") if thr is not None else 0,
            _lib.ptr(out), out.stride(0), out.stride(1), _lib.dtype_code(out, "out"),
            _lib.ptr(row_nnz), M, N, K, act, None, _lib.stream(dev))


def test_noalloc_encode_equals_sf_encode_on_two_calls():
    sae, x, meta = workloads.make("C3", T=4096, d_sae=16384, device="cuda")  # JumpReLU, bf16, d_in 2304
    for T in (4096, 1000):
        xs = x[:T]
        want_nnz = torch.zeros(T, device="cuda", dtype=torch.int32)
        want = fused_encode(xs, sae.W_enc, sae.b_enc, sae.b_dec, sae.threshold, "jumprelu", row_nnz=want_nnz)
        out = torch.full_like(want, float("nan"))
        nnz = torch.zeros(T, device="cuda", dtype=torch.int32)
        rc = encode_noalloc(xs, sae.W_enc, sae.b_enc, sae.b_dec, sae.threshold, 1, out, nnz)
        assert rc == _lib.SF_OK, _lib.load().sf_last_error()
        torch.cuda.synchronize()
        assert torch.equal(out, want)
        assert torch.equal(nnz, want_nnz)
        assert int(nnz.sum()) > 0


def test_noalloc_encode_runs_token_counts_beyond_its_array_in_chunks():
    sae, x, meta = workloads.make("C3", T=16384, d_sae=512, device="cuda")  # d_in 2304 bf16: 7168 rows a chunk
    assert 16384 * 2304 * 2 > (32 << 20)
    for T in (16384, 7169, 7168, 300):  # 3 chunks (the last ragged), 2 (one row in the second), 1, 1
        xs = x[:T]
        want_nnz = torch.zeros(T, device="cuda", dtype=torch.int32)
        want = fused_encode(xs, sae.W_enc, sae.b_enc, sae.b_dec, sae.threshold, "jumprelu", row_nnz=want_nnz)
        out = torch.full_like(want, float("nan"))
        nnz = torch.zeros(T, device="cuda", dtype=torch.int32)
        rc = encode_noalloc(xs, sae.W_enc, sae.b_enc, sae.b_dec, sae.threshold, 1, out, nnz)
        assert rc == _lib.SF_OK, _lib.load().sf_last_error()
        torch.cuda.synchronize()
        assert torch.equal(out, want), T
        assert torch.equal(nnz, want_nnz), T


def test_noalloc_encode_refuses_a_d_in_beyond_its_array():
    K = 65664  # 256 rows x 65664 x 2 B of x' exceed the 32 MiB array
    x = torch.randn(300, K, device="cuda").to(torch.bfloat16)
    W = torch.zeros(K, 256, device="cuda", dtype=torch.bfloat16)
    b_enc = torch.zeros(256, device="cuda", dtype=torch.bfloat16)
    b_dec = torch.zeros(K, device="cuda", dtype=torch.bfloat16)
    out = torch.full((300, 256), 7.0, device="cuda", dtype=torch.bfloat16)
    rc = encode_noalloc(x, W, b_enc, b_dec, None, 0, out, None)
    assert rc == _lib.SF_EINVAL
    assert b"scratch array" in _lib.load().sf_last_error()
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())  # nothing was launched
    # the next call still works
    sae, xs, meta = workloads.make("C3", T=1000, d_sae=512, device="cuda")
    out2 = torch.empty(1000, 512, device="cuda", dtype=torch.bfloat16)
    rc = encode_noalloc(xs, sae.W_enc, sae.b_enc, sae.b_dec, None, 0, out2, None)
    assert rc == _lib.SF_OK
    torch.testing.assert_close(out2, fused_encode(xs, sae.W_enc, sae.b_enc, sae.b_dec), rtol=0, atol=0)
