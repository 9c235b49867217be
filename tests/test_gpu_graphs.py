"""GPU: the launch paths that make no host read replay from a HIP graph.

fused_encode, sparse_decode and the whole TopK forward (encode_sparse's row-candidate select,
its on-device redo of overflowed rows, and decode_sparse) launch hand-written kernels through
the C ABI on torch's current stream with no host sync and no allocation of their own, so a
serving loop can capture them once and replay them. Each test captures a path, then replays it
several times with new inputs written eagerly between the replays and other eager work in
between, and checks every replay bit for bit against the same path run eagerly.
"""

import pytest
import torch

import saeflow_amd
from saeflow_amd import ops, workloads
from saeflow_amd.kernels import best_config, fused_encode, sparse_decode
from saeflow_amd.kernels import encode as kenc

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.view(torch.int32) if t.dtype == torch.float32 else t.view(torch.int16)


def _capture(fn):
    """fn() run once on a side stream (warm-up, as torch.cuda.graphs recommends), then captured."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


def _sae(d_in, d_sae, activation, dtype, k=None, seed=0):
    torch.manual_seed(seed)
    sae = saeflow_amd.SAE(d_in, d_sae, activation, k=k, device="cuda", dtype=dtype)
    with torch.no_grad():
        sae.W_enc.mul_(3.0)
        sae.b_enc.copy_(torch.randn(d_sae, device="cuda") * 0.1)
        sae.b_dec.copy_(torch.randn(d_in, device="cuda") * 0.1)
    return sae


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_dense_encode_and_decode_replay_from_a_graph(dtype):
    M, d_in, d_sae = 300, 128, 2000
    sae = _sae(d_in, d_sae, "relu", dtype)
    x = torch.randn(M, d_in, device="cuda").to(dtype)
    # a fixed CSR for the decode: 24 features per token
    indices = torch.randint(0, d_sae, (M * 24,), device="cuda", dtype=torch.int32)
    values = torch.randn(M * 24, device="cuda").to(dtype)
    indptr = torch.arange(0, M * 24 + 1, 24, device="cuda", dtype=torch.int64)
    row_nnz = torch.zeros(M, device="cuda", dtype=torch.int32)

    def path():
        row_nnz.zero_()
        f = fused_encode(x, sae.W_enc, sae.b_enc, sae.b_dec, row_nnz=row_nnz)
        out = sparse_decode(indptr, indices, values, sae.W_dec, sae.b_dec)
        return f, out

    g, (f_g, out_g) = _capture(path)
    for i in range(4):
        x.copy_(torch.randn(M, d_in, device="cuda").to(dtype))
        values.copy_(torch.randn(M * 24, device="cuda").to(dtype))
        torch.randn(1 << 20, device="cuda").sum()  # unrelated eager work between the replays
        g.replay()
        torch.cuda.synchronize()
        got_f, got_out, got_cnt = f_g.clone(), out_g.clone(), row_nnz.clone()
        want_f, want_out = path()
        assert torch.equal(_bits(got_f), _bits(want_f)), i
        assert torch.equal(got_cnt, row_nnz), i
        assert torch.equal(_bits(got_out), _bits(want_out)), i


@pytest.mark.parametrize("d_sae", [20000, 3000])  # the row-candidate select, the dense select
def test_topk_forward_replays_from_a_graph(d_sae):
    M, d_in, k = 300, 128, 16
    sae = _sae(d_in, d_sae, "topk", torch.bfloat16, k=k)
    x = torch.randn(M, d_in, device="cuda").to(torch.bfloat16)
    row_path = d_sae >= ops.TOPK_MIN_FEATURES

    def path():
        csr = saeflow_amd.encode_sparse(sae, x)
        return csr, saeflow_amd.decode_sparse(sae, csr)

    g, ((indptr_g, idx_g, val_g), xh_g) = _capture(path)
    for i in range(4):
        x.copy_(torch.randn(M, d_in, device="cuda").to(torch.bfloat16))
        if i == 2 and row_path:
            x[7] = float("nan")  # a NaN token overflows its candidate list: the on-device redo runs
        torch.randn(1 << 20, device="cuda").sum()
        g.replay()
        torch.cuda.synchronize()
        got = (indptr_g.clone(), idx_g.clone(), val_g.clone(), xh_g.clone())
        (indptr, idx, val), xh = path()
        assert torch.equal(got[0], indptr), i
        assert torch.equal(got[1], idx), i
        assert torch.equal(_bits(got[2]), _bits(val)), i
        assert torch.equal(_bits(got[3]), _bits(xh)), i
        if i == 2 and row_path:  # the redo ran: the all-NaN row's top-k is its first k columns
            assert got[1].view(M, k)[7].tolist() == list(range(k))


def test_captured_encode_keeps_the_autotuned_tiling():
    # A shape large enough to autotune: the eager call times the tilings; under capture no timing
    # runs and the shape's pick is reused, so the graph's launches are those of the eager path.
    sae, x, meta = workloads.make("C2", T=4096, device="cuda")
    kenc._tuned.clear()
    row_nnz = torch.zeros(4096, device="cuda", dtype=torch.int32)

    def path():
        row_nnz.zero_()
        return fused_encode(x, sae.W_enc, sae.b_enc, sae.b_dec, sae.threshold, "jumprelu", row_nnz=row_nnz)

    want = path().clone()
    picked = best_config()
    assert len(kenc._tuned) == 1 and picked in kenc._candidates(torch.bfloat16)
    g, f_g = _capture(path)
    assert best_config() == picked
    for _ in range(3):
        torch.randn(1 << 20, device="cuda").sum()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(_bits(f_g), _bits(want))
        assert torch.equal(row_nnz, torch.count_nonzero(want, dim=1).int())
