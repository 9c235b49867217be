"""CPU: the oracle is pinned before it is trusted.

Each oracle function is checked against (a) the committed golden fixtures (written from
element-by-element float64 brute force), (b) brute force on fresh tiny inputs, (c) a
library routine where one exists (torch.Tensor.to_sparse_csr, torch.topk, a dense matmul),
and (d) known answers; planted mistakes show that these checks catch plausible errors.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import brute, csr, reference

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def t(a):
    return torch.from_numpy(np.asarray(a))


# ----------------------------------------------------------------------------- encode


@pytest.mark.parametrize("name", ["encode_relu", "encode_jumprelu", "encode_topk", "encode_relu_bf16"])
def test_encode_matches_golden(name):
    g = load(name)
    act, k = str(g["activation"]), int(g["k"]) or None
    pre = reference.encode_pre(t(g["x"]), t(g["W_enc"]), t(g["b_enc"]), t(g["b_dec"]), dtype=torch.float64)
    np.testing.assert_allclose(pre.numpy(), g["pre"], rtol=1e-12, atol=1e-12)
    out = reference.encode(t(g["x"]), t(g["W_enc"]), t(g["b_enc"]), t(g["b_dec"]), t(g["threshold"]), act, k,
                           dtype=torch.float64)
    np.testing.assert_allclose(out.numpy(), g["out"], rtol=1e-12, atol=1e-12)
    out32 = reference.encode(t(g["x"]), t(g["W_enc"]), t(g["b_enc"]), t(g["b_dec"]), t(g["threshold"]), act, k)
    np.testing.assert_allclose(out32.numpy(), g["out"], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("activation", ["relu", "jumprelu", "topk"])
def test_encode_matches_brute_force(activation):
    gen = torch.Generator().manual_seed(5)
    M, K, N = 4, 7, 11
    x, W = torch.randn(M, K, generator=gen), torch.randn(K, N, generator=gen)
    b_enc, b_dec, thr = torch.randn(N, generator=gen), torch.randn(K, generator=gen), torch.rand(N, generator=gen)
    pre, want = brute.encode(x.double().tolist(), W.double().tolist(), b_enc.double().tolist(),
                             b_dec.double().tolist(), thr.double().tolist(), activation, 4)
    got = reference.encode(x, W, b_enc, b_dec, thr, activation, 4, dtype=torch.float64)
    np.testing.assert_allclose(got.numpy(), np.array(want), rtol=1e-12, atol=1e-12)


def test_encode_pre_is_a_textbook_affine_map():
    # linearity in x: encode_pre(x1 + x2) - encode_pre(x2) = x1 @ W + b_dec @ W ... spelled out:
    gen = torch.Generator().manual_seed(6)
    x1, x2 = torch.randn(3, 8, generator=gen, dtype=torch.float64), torch.randn(3, 8, generator=gen,
                                                                                dtype=torch.float64)
    W, b_enc, b_dec = (torch.randn(8, 5, generator=gen, dtype=torch.float64), torch.randn(5, generator=gen,
                       dtype=torch.float64), torch.randn(8, generator=gen, dtype=torch.float64))
    f = lambda x: reference.encode_pre(x, W, b_enc, b_dec, dtype=torch.float64)  # noqa: E731
    torch.testing.assert_close(f(x1 + x2) - f(x2), x1 @ W)
    # b_dec enters with a minus sign, b_enc with a plus sign
    torch.testing.assert_close(f(b_dec.expand(2, 8)), b_enc.expand(2, 5))


def test_ops_topk_relu_first_equals_reference_topk_on_dense_view():
    gen = torch.Generator().manual_seed(8)
    x, W = torch.randn(6, 10, generator=gen), torch.randn(10, 40, generator=gen)
    b_enc, b_dec = torch.randn(40, generator=gen), torch.randn(10, generator=gen)
    top = reference.ops_topk(x, W, b_enc, b_dec, 5)
    dense = torch.zeros(6, 40).scatter_(-1, top.indices, top.values)
    torch.testing.assert_close(dense, reference.encode(x, W, b_enc, b_dec, None, "topk", 5))


# ----------------------------------------------------------------------------- dense -> CSR


def test_dense_to_csr_matches_golden():
    g = load("csr")
    indptr, indices, values = csr.dense_to_csr(t(g["f"]))
    np.testing.assert_array_equal(indptr, g["indptr"])
    np.testing.assert_array_equal(indices, g["indices"])
    np.testing.assert_array_equal(values.numpy(), g["values"])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(1, 32), (37, 129), (64, 300)])
def test_dense_to_csr_matches_torch_bit_exact(shape, dtype):
    f = torch.relu(torch.randn(*shape) - 1.0).to(dtype)
    f[0] = 0
    indptr, indices, values = csr.dense_to_csr(f)
    want = f.to_sparse_csr()
    np.testing.assert_array_equal(indptr, want.crow_indices().numpy())
    np.testing.assert_array_equal(indices, want.col_indices().numpy())
    assert torch.equal(values.view(torch.int16 if dtype != torch.float32 else torch.int32),
                       want.values().view(torch.int16 if dtype != torch.float32 else torch.int32))


def test_dense_to_csr_matches_brute_force():
    f = torch.relu(torch.randn(9, 17) - 0.5)
    f[2] = 0
    ip, ix, vals = brute.dense_to_csr(f.double().tolist())
    indptr, indices, values = csr.dense_to_csr(f)
    assert indptr.tolist() == ip and indices.tolist() == ix
    np.testing.assert_array_equal(values.double().numpy(), np.array(vals))


def test_dense_to_csr_known_answers():
    indptr, indices, values = csr.dense_to_csr(torch.zeros(5, 40))
    assert indptr.tolist() == [0] * 6 and indices.size == 0 and values.numel() == 0
    f = torch.tensor([[0.0, -0.0, 1.5], [float("nan"), 0.0, 0.0]])
    indptr, indices, values = csr.dense_to_csr(f)
    assert indptr.tolist() == [0, 1, 2] and indices.tolist() == [2, 0]
    assert values[0] == 1.5 and torch.isnan(values[1])


def test_csr_round_trip_and_row_counts():
    f = torch.relu(torch.randn(13, 50) - 1.0)
    indptr, indices, values = csr.dense_to_csr(f)
    np.testing.assert_array_equal(csr.csr_to_dense(indptr, indices, values.numpy(), 50), f.double().numpy())
    np.testing.assert_array_equal(np.diff(indptr), csr.row_counts(f))


# ----------------------------------------------------------------------------- decode


def test_decode_matches_golden():
    g = load("decode")
    out = csr.sparse_decode(g["indptr"], g["indices"], g["values"], g["W_dec"], g["b_dec"])
    np.testing.assert_allclose(out, g["out"], rtol=1e-12, atol=1e-12)


def test_decode_equals_dense_matmul_and_brute_force():
    gen = torch.Generator().manual_seed(9)
    f = torch.relu(torch.randn(7, 30, generator=gen, dtype=torch.float64) - 1.5)
    W, b = torch.randn(30, 12, generator=gen, dtype=torch.float64), torch.randn(12, generator=gen,
                                                                               dtype=torch.float64)
    indptr, indices, values = csr.dense_to_csr(f)
    got = csr.sparse_decode(indptr, indices, values.numpy(), W.numpy(), b.numpy())
    np.testing.assert_allclose(got, (f @ W + b).numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(got, reference.decode(f, W, b, dtype=torch.float64).numpy(), rtol=1e-12, atol=1e-12)
    want = brute.sparse_decode(indptr.tolist(), indices.tolist(), values.tolist(), W.tolist(), b.tolist())
    np.testing.assert_allclose(got, np.array(want), rtol=1e-12, atol=1e-12)


# ----------------------------------------------------------------------------- top-k


def test_topk_matches_golden_tie_rule():
    g = load("topk")
    vals, cols = csr.topk_rows(g["f"], int(g["k"]))
    np.testing.assert_array_equal(vals, g["values"])
    np.testing.assert_array_equal(cols, g["cols"])
    # ties resolved by increasing column: row 0 keeps 3.0 then the 2.0s at columns 1, 2
    assert cols[0].tolist() == [4, 1, 2]


def test_topk_matches_torch_values():
    f = torch.randn(20, 300)
    vals, cols = csr.topk_rows(f.numpy(), 17)
    top = f.topk(17, dim=-1)
    np.testing.assert_array_equal(vals, top.values.double().numpy())
    np.testing.assert_array_equal(cols, top.indices.numpy())  # no ties in continuous data


def test_topk_zero_signs_and_nans_match_torch():
    """-0.0 and +0.0 tie (so columns decide) and NaNs of either sign rank first, as in
    torch.topk; the values agree with torch.topk's (NaN where torch has NaN)."""
    f = torch.tensor([[0.0, -0.0, 1.0, -0.0, 0.0, -1.0],
                      [2.0, float("nan"), 3.0, -float("nan"), 1.0, float("inf")],
                      [-0.0, -0.0, -0.0, 0.0, 0.0, 0.0]])
    for k in (1, 3, 6):
        vals, cols = csr.topk_rows(f.numpy(), k)
        top = f.topk(k, dim=-1)
        np.testing.assert_array_equal(vals, top.values.double().numpy())  # NaN == NaN here
    vals, cols = csr.topk_rows(f.numpy(), 6)
    assert cols[0].tolist() == [2, 0, 1, 3, 4, 5]  # zeros of both signs by column
    assert cols[1].tolist() == [1, 3, 5, 2, 0, 4]  # NaNs first (by column), then +inf
    assert cols[2].tolist() == [0, 1, 2, 3, 4, 5]
    # a planted order that ranks +0.0 above -0.0 (the raw sign-magnitude key) is caught
    row = f[0].numpy()
    planted = np.lexsort((np.arange(6), np.signbit(row), -row))
    assert planted.tolist() == [2, 0, 4, 1, 3, 5] != cols[0].tolist()


# ----------------------------------------------------------------------------- planted mistakes


def test_planted_mistakes_are_caught():
    g = load("encode_jumprelu")
    x, W, b_enc, b_dec, thr = (t(g[k]) for k in ("x", "W_enc", "b_enc", "b_dec", "threshold"))
    want = g["out"]

    def differs(out):
        return not np.allclose(out, want, rtol=1e-9, atol=1e-9)

    d = torch.float64
    x, W, b_enc, b_dec, thr = (v.to(d) for v in (x, W, b_enc, b_dec, thr))
    assert differs(torch.relu(((x + b_dec) @ W + b_enc)) * (((x + b_dec) @ W + b_enc) > thr))  # b_dec sign
    assert differs(torch.relu((x - b_dec) @ W) * (((x - b_dec) @ W) > thr))                      # dropped b_enc
    pre = (x - b_dec) @ W + b_enc
    assert differs(torch.relu(pre) * (pre > -thr))                                                # threshold sign
    assert differs(torch.relu(pre))                                                               # relu for jumprelu
    W2 = torch.roll(W, 1, dims=0)
    assert differs(torch.relu((x - b_dec) @ W2 + b_enc) * (((x - b_dec) @ W2 + b_enc) > thr))    # wrong W row index

    gc = load("csr")
    indptr = gc["indptr"].copy()
    indptr[1:] = indptr[:-1]  # shifted indptr
    assert not np.array_equal(indptr, gc["indptr"])
    gd = load("decode")
    bad = csr.sparse_decode(gd["indptr"], gd["indices"], gd["values"], gd["W_dec"][::-1].copy(), gd["b_dec"])
    assert not np.allclose(bad, gd["out"])
    gt = load("topk")
    f = gt["f"][:, ::-1].copy()  # reversed columns flip the tie order
    vals, cols = csr.topk_rows(f, 3)
    assert not np.array_equal(f.shape[1] - 1 - cols, gt["cols"])


# ----------------------------------------------------------------------------- backward
def _backward_case(seed=0, M=4, D=5, N=7):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)  # noqa: E731
    x, W_enc, b_enc, W_dec, b_dec = r(M, D), r(D, N), r(N), r(N, D), r(D)
    active = torch.rand(M, N, generator=g) < 0.4
    return x, W_enc, b_enc, W_dec, b_dec, active, r(M, D), r(M, N)


def _loss(x, W_enc, b_enc, W_dec, b_dec, active, G, H):
    f = ((x - b_dec) @ W_enc + b_enc) * active
    return float(((f @ W_dec + b_dec) * G).sum() + (f * H).sum())


def test_backward_oracle_matches_finite_differences():
    from oracle import backward
    case = _backward_case()
    got = backward.grads(*case)
    params = list(case[:5])
    eps = 1e-6
    for i, name in enumerate(["x", "W_enc", "b_enc", "W_dec", "b_dec"]):
        fd = torch.zeros_like(params[i])
        flat = params[i].view(-1)
        for k in range(flat.numel()):
            old = flat[k].item()
            flat[k] = old + eps
            up = _loss(*params, *case[5:])
            flat[k] = old - eps
            dn = _loss(*params, *case[5:])
            flat[k] = old
            fd.view(-1)[k] = (up - dn) / (2 * eps)
        torch.testing.assert_close(got[name], fd, atol=1e-6, rtol=1e-6, msg=name)


def test_backward_oracle_closed_forms_and_planted_mistakes():
    from oracle import backward
    x, W_enc, b_enc, W_dec, b_dec, active, G, H = _backward_case(seed=1, M=6, D=4, N=9)
    got = backward.grads(x, W_enc, b_enc, W_dec, b_dec, active, G, H)
    f = ((x - b_dec) @ W_enc + b_enc) * active
    g_pre = (G @ W_dec.T + H) * active
    torch.testing.assert_close(got["W_dec"], f.T @ G)
    torch.testing.assert_close(got["b_enc"], g_pre.sum(0))
    torch.testing.assert_close(got["W_enc"], (x - b_dec).T @ g_pre)
    torch.testing.assert_close(got["x"], g_pre @ W_enc.T)
    torch.testing.assert_close(got["b_dec"], G.sum(0) - (g_pre @ W_enc.T).sum(0))
    # plausible mistakes are caught by these closed forms
    assert not torch.allclose(got["W_enc"], (x + b_dec).T @ g_pre)  # sign of b_dec
    assert not torch.allclose(got["b_dec"], G.sum(0))  # the encoder's share dropped
    assert not torch.allclose(got["b_enc"], (G @ W_dec.T).mul(active).sum(0))  # dL/df dropped
