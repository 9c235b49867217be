"""GPU: the backward kernels of the sparse path against float64 autograd of the forward.

The reference has no backward (README.md:244 lists it on the roadmap); the oracle is the
mathematics of its forward (reference.py:36-52) differentiated by torch autograd in float64
on the nonzero set the GPU encode produced (oracle/backward.py), itself pinned by finite
differences in tests/test_oracle.py.

Tolerances (stated per dtype, relative to each gradient's largest magnitude): fp32 1e-4,
fp16 1e-2, bf16 3e-2. The kernels accumulate in fp32; the differences from the float64
oracle come from the forward's rounded features and x' = cast(x - b_dec), and from rounding
the gradients to the parameters' dtype. The CSR -> CSC transpose is compared exactly.
"""

import numpy as np
import pytest
import torch

import saeflow_amd
from oracle import backward as obwd
from saeflow_amd.kernels import csr_to_dense
from saeflow_amd.kernels.backward import csr_transpose, sparse_backward
from saeflow_amd.training import forward_train

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-4, torch.float16: 1e-2, torch.bfloat16: 3e-2}


class Sae:
    def __init__(self, **kw):
        self.__dict__.update(kw)


def make(M, D, N, activation, dtype, seed=0, hot=0, k=8):
    """The reference test recipe (test_kernels.py:14-20) on the CPU, then rounded to dtype;
    `hot` features get b_enc = +4 so they fire on every token (columns of M entries)."""
    g = torch.Generator().manual_seed(seed)
    W_dec = torch.randn(N, D, generator=g)
    W_dec /= W_dec.norm(dim=1, keepdim=True)
    b_enc = torch.randn(N, generator=g) * 0.1 - 0.5
    b_enc[:hot] = 4.0
    p = dict(W_dec=W_dec, W_enc=W_dec.T.contiguous(), b_enc=b_enc, b_dec=torch.randn(D, generator=g) * 0.1,
             threshold=torch.rand(N, generator=g) * 0.5 if activation == "jumprelu" else None)
    p = {key: (v.to(dtype) if v is not None else None) for key, v in p.items()}
    x = torch.randn(M, D, generator=g).to(dtype)
    return p, x, Sae(activation=activation, k=k if activation == "topk" else None, **{key: (v.cuda() if v is not None else None) for key, v in p.items()})


def check(name, got, want, dtype):
    got = got.detach().double().cpu()
    scale = float(want.abs().max()) if want.numel() else 0.0
    torch.testing.assert_close(got, want, atol=TOL[dtype] * max(scale, 1e-30), rtol=TOL[dtype], msg=name)


def run_case(M, D, N, activation, dtype, hot=0, seed=0, with_h=True):
    p, x, sae = make(M, D, N, activation, dtype, seed=seed, hot=hot)
    xg = x.cuda()
    indptr, indices, values = saeflow_amd.encode_sparse(sae, xg)
    g = torch.Generator().manual_seed(seed + 1)
    G = torch.randn(M, D, generator=g).to(dtype)
    H = torch.randn(indices.numel(), generator=g).to(dtype) if with_h else None
    got = sparse_backward(xg, sae.W_enc, sae.b_enc, sae.W_dec, sae.b_dec, (indptr, indices, values), G.cuda(),
                          None if H is None else H.cuda())
    ones = torch.ones(indices.numel(), dtype=torch.float32, device="cuda")
    pattern = csr_to_dense(indptr, indices, ones, N).cpu()
    # the derivative is 1 where the stored feature is positive (topk rows may hold zeros)
    f_gpu = csr_to_dense(indptr, indices, values, N).double().cpu()
    active = (pattern > 0) & (f_gpu > 0)
    Hd = None
    if H is not None:
        Hd = csr_to_dense(indptr, indices, H.cuda().float(), N).cpu()
    want = obwd.grads(x, p["W_enc"], p["b_enc"], p["W_dec"], p["b_dec"], active, G, Hd)
    return got, want, (indptr, indices, values)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("activation", ["relu", "jumprelu", "topk"])
@pytest.mark.parametrize("shape", [(64, 64, 256), (37, 50, 129), (300, 128, 520), (700, 72, 96)])
def test_sparse_backward_matches_oracle(shape, activation, dtype):
    M, D, N = shape
    got, want, _ = run_case(M, D, N, activation, dtype, hot=3 if M > 256 else 0)
    for name in ("W_enc", "b_enc", "W_dec", "b_dec", "x"):
        check(name, getattr(got, name), want[name], dtype)


def test_sparse_backward_is_deterministic_with_long_columns():
    """Columns longer than one work item (3 features fire on all 1500 tokens) are summed from
    fp32 partials in a fixed order: two calls give identical bits."""
    p, x, sae = make(1500, 256, 384, "relu", torch.bfloat16, hot=3)
    xg = x.cuda()
    csr = saeflow_amd.encode_sparse(sae, xg)
    G = torch.randn(1500, 256, device="cuda").to(torch.bfloat16)
    a = sparse_backward(xg, sae.W_enc, sae.b_enc, sae.W_dec, sae.b_dec, csr, G)
    b = sparse_backward(xg, sae.W_enc, sae.b_enc, sae.W_dec, sae.b_dec, csr, G)
    for name in ("W_enc", "b_enc", "W_dec", "b_dec", "x", "pre"):
        ta, tb = getattr(a, name), getattr(b, name)
        assert torch.equal(ta.view(torch.int16) if ta.dtype == torch.bfloat16 else ta,
                           tb.view(torch.int16) if tb.dtype == torch.bfloat16 else tb), name
    counts = torch.bincount(csr[1].long(), minlength=384)
    assert int(counts[:3].min()) == 1500  # the long columns exist


def _csc_numpy(indptr, indices, N):
    indptr, indices = indptr.cpu().numpy(), indices.cpu().numpy()
    rows = np.repeat(np.arange(len(indptr) - 1), np.diff(indptr))
    pos = np.arange(len(indices))
    ok = (indices >= 0) & (indices < N)
    order = np.lexsort((pos[ok], rows[ok], indices[ok]))
    colptr = np.zeros(N + 1, dtype=np.int64)
    colptr[1:] = np.cumsum(np.bincount(indices[ok], minlength=N))
    return colptr, rows[ok][order], pos[ok][order]


@pytest.mark.parametrize("M,N", [(300, 500), (5000, 64)])
def test_csr_transpose_exact(M, N):
    """Columns of 0, 1, <= 64 and many entries; invalid indices are left out."""
    g = torch.Generator().manual_seed(M)
    dense = torch.rand(M, N, generator=g) < 0.05
    dense[:, 7] = True  # a column with an entry in every row
    dense[:, 11] = False  # an empty column
    indptr = torch.zeros(M + 1, dtype=torch.int64)
    indptr[1:] = torch.cumsum(dense.sum(1), 0)
    indices = torch.nonzero(dense)[:, 1].int()
    indices[::97] = -3  # invalid entries
    indices[5::211] = N + 4
    colptr, rows, pos = csr_transpose(indptr.cuda(), indices.cuda(), N)
    want = _csc_numpy(indptr, indices, N)
    np.testing.assert_array_equal(colptr.cpu().numpy(), want[0])
    n = int(want[0][-1])
    np.testing.assert_array_equal(rows.cpu().numpy()[:n], want[1])
    np.testing.assert_array_equal(pos.cpu().numpy()[:n], want[2])


@pytest.mark.parametrize("M,N,maxlen,canonical,empty", [
    (1, 70000, 4000, True, 0.0),  # one row of thousands of entries
    (40000, 3, 4, False, 0.5),  # one column per bucket, repeats, 32 rows per wave
    (3000, 1 << 20, 200, True, 0.3),  # the widest headline configuration
    (700, 12345, 150, False, 0.9),  # unsorted rows, long runs of empty rows
    (50, 1 << 23, 40, True, 0.0),  # the widest the counting sort takes (4096 buckets)
    (100, (1 << 23) + 1, 50, True, 0.0),  # beyond 2^23 columns: the fallback path
])
def test_csr_transpose_random_shapes(M, N, maxlen, canonical, empty):
    """Random row lengths (empty rows included), canonical or unsorted rows with repeats,
    invalid indices: colptr, rows and positions equal a stable sort by column on the CPU."""
    rng = np.random.default_rng(M + N)
    lens = rng.integers(0, maxlen + 1, M) * (rng.random(M) >= empty)
    indptr = np.zeros(M + 1, dtype=np.int64)
    indptr[1:] = np.cumsum(lens)
    cols = []
    for n in lens:
        c = rng.integers(0, N, n)
        cols.append(np.unique(c) if canonical else c)
    lens = np.array([len(c) for c in cols])
    indptr[1:] = np.cumsum(lens)
    indices = np.concatenate(cols).astype(np.int32) if M else np.zeros(0, np.int32)
    bad = rng.random(indices.size) < 0.01
    indices[bad] = rng.choice(np.array([-1, N, N + 7, -(1 << 30)], dtype=np.int32), int(bad.sum()))
    ip, ix = torch.from_numpy(indptr), torch.from_numpy(indices)
    colptr, rows, pos = csr_transpose(ip.cuda(), ix.cuda(), N)
    want = _csc_numpy(ip, ix, N)
    np.testing.assert_array_equal(colptr.cpu().numpy(), want[0])
    n = int(want[0][-1])
    np.testing.assert_array_equal(rows.cpu().numpy()[:n], want[1])
    np.testing.assert_array_equal(pos.cpu().numpy()[:n], want[2])


def test_csr_transpose_with_repeated_columns():
    """A CSR row that names one column twice (non-canonical input) still fills every CSC
    slot exactly once, ordered by row then CSR position."""
    M, N = 200, 4  # columns of ~125 entries, so the bitmap path meets the repeats
    g = torch.Generator().manual_seed(5)
    lens = torch.randint(0, 6, (M,), generator=g)
    indptr = torch.zeros(M + 1, dtype=torch.int64)
    indptr[1:] = torch.cumsum(lens, 0)
    indices = torch.randint(0, N, (int(indptr[-1]),), generator=g).int()  # repeats within rows
    indices[indptr[10]:indptr[11]] = 3
    colptr, rows, pos = csr_transpose(indptr.cuda(), indices.cuda(), N)
    want = _csc_numpy(indptr, indices, N)
    np.testing.assert_array_equal(colptr.cpu().numpy(), want[0])
    np.testing.assert_array_equal(rows.cpu().numpy(), want[1])
    np.testing.assert_array_equal(pos.cpu().numpy(), want[2])


def test_forward_train_autograd_matches_oracle():
    """loss.backward() through forward_train fills every parameter's grad (and x.grad) with
    the oracle's gradients of the same loss: squared reconstruction error plus an L1 penalty
    on the feature values."""
    M, D, N = 96, 64, 320
    p, x, _ = make(M, D, N, "jumprelu", torch.float32, seed=3)
    leaves = {key: v.cuda().requires_grad_(key != "threshold") for key, v in p.items()}
    sae = Sae(activation="jumprelu", k=None, **leaves)
    xg = x.cuda().requires_grad_(True)
    x_hat, (indptr, indices, values) = forward_train(sae, xg)
    lam = 0.05
    loss = (x_hat - xg.detach()).pow(2).sum() + lam * values.abs().sum()
    loss.backward()
    active = csr_to_dense(indptr, indices, torch.ones_like(values), N).cpu() > 0
    G = 2 * (x_hat - xg).detach().cpu()
    Hd = csr_to_dense(indptr, indices, lam * torch.sign(values).detach(), N).cpu()
    want = obwd.grads(x, p["W_enc"], p["b_enc"], p["W_dec"], p["b_dec"], active, G, Hd)
    for name in ("W_enc", "b_enc", "W_dec", "b_dec"):
        check(name, leaves[name].grad, want[name], torch.float32)
    check("x", xg.grad, want["x"], torch.float32)
    assert leaves["threshold"].grad is None


def test_sparse_backward_without_nonzeros_and_without_rows():
    p, x, sae = make(40, 32, 48, "relu", torch.float32)
    sae.b_enc = torch.full_like(sae.b_enc, -100.0)  # nothing fires
    xg = x.cuda()
    csr = saeflow_amd.encode_sparse(sae, xg)
    assert csr[1].numel() == 0
    G = torch.randn(40, 32, device="cuda")
    got = sparse_backward(xg, sae.W_enc, sae.b_enc, sae.W_dec, sae.b_dec, csr, G)
    assert float(got.W_enc.abs().max()) == 0 and float(got.W_dec.abs().max()) == 0
    assert float(got.b_enc.abs().max()) == 0 and float(got.x.abs().max()) == 0
    torch.testing.assert_close(got.b_dec, G.sum(0), atol=1e-5, rtol=1e-5)
    empty = (torch.zeros(1, dtype=torch.int64, device="cuda"), torch.zeros(0, dtype=torch.int32, device="cuda"),
             torch.zeros(0, device="cuda"))
    got0 = sparse_backward(xg[:0], sae.W_enc, sae.b_enc, sae.W_dec, sae.b_dec, empty, G[:0])
    assert got0.x.shape == (0, 32) and float(got0.W_enc.abs().max()) == 0 and float(got0.b_dec.abs().max()) == 0


def test_input_gradient_is_optional():
    """need_grad_x=False skips dx' (the decode over W_enc^T) and changes nothing else."""
    p, x, sae = make(300, 128, 520, "jumprelu", torch.bfloat16, hot=3)
    xg = x.cuda()
    csr = saeflow_amd.encode_sparse(sae, xg)
    G = torch.randn(300, 128, device="cuda").to(torch.bfloat16)
    a = sparse_backward(xg, sae.W_enc, sae.b_enc, sae.W_dec, sae.b_dec, csr, G)
    b = sparse_backward(xg, sae.W_enc, sae.b_enc, sae.W_dec, sae.b_dec, csr, G, need_grad_x=False)
    assert a.x is not None and b.x is None
    for name in ("W_enc", "b_enc", "W_dec", "b_dec", "pre"):
        ta, tb = getattr(a, name), getattr(b, name)
        assert torch.equal(ta.float(), tb.float()), name


@pytest.mark.parametrize("name", ["C3", "C5"])
def test_backward_at_full_size_on_sampled_features(name):
    """The headline configuration C3 (T = 16384, d_sae = 65536) and C5 at its real width
    (d_sae = 2^20, W_enc / W_dec 4.8 GB each; T = 4096): the backward's gradients of sampled
    features checked against their closed forms in float64 from the GPU's own CSR
    (dW_dec[j] = sum_m f[m,j] G[m], dW_enc[:, j] = sum_m g_pre[m,j] x'[m], db_enc[j] =
    sum_m g_pre[m,j]), dL/dpre on sampled entries against G[m] . W_dec[j], unused features
    exactly zero, and db_dec against colsum(G) - W_enc db_enc."""
    from saeflow_amd import workloads
    sae, x, meta = workloads.make(name, device="cuda")
    M, D = x.shape
    N = sae.W_enc.shape[1]
    indptr, indices, values = saeflow_amd.encode_sparse(sae, x)
    g = torch.Generator(device="cuda").manual_seed(7)
    G = torch.randn(M, D, device="cuda", generator=g).to(torch.bfloat16)
    got = sparse_backward(x, sae.W_enc, sae.b_enc, sae.W_dec, sae.b_dec, (indptr, indices, values), G,
                          need_grad_x=False)
    tol = TOL[torch.bfloat16]
    counts = torch.bincount(indices.long(), minlength=N)
    used = torch.nonzero(counts).flatten()
    hot = int(torch.argmax(counts))
    js = torch.cat([used[:: max(1, used.numel() // 6)][:6].cpu(), torch.tensor([hot, N - 1])])
    rows_of = torch.repeat_interleave(torch.arange(M, device="cuda"), indptr[1:] - indptr[:-1])
    xs = (x.double() - sae.b_dec.double()).to(torch.bfloat16).double()  # x' as the forward used it
    for j in js.tolist():
        sel = indices == j
        ms, fv, gp = rows_of[sel], values[sel].double(), got.pre[sel].double()
        want_dec = (fv[:, None] * G[ms].double()).sum(0)
        want_enc = (gp[:, None] * xs[ms]).sum(0)
        check(f"W_dec[{j}]", got.W_dec[j], want_dec.cpu(), torch.bfloat16)
        check(f"W_enc[:, {j}]", got.W_enc[:, j], want_enc.cpu(), torch.bfloat16)
        torch.testing.assert_close(got.b_enc[j].double().cpu(), gp.sum().cpu(), atol=1e-3 * (1 + gp.abs().sum().item()),
                                   rtol=1e-3)
    # dL/dpre on sampled entries: G[m] . W_dec[j] (no penalty term here)
    e = torch.tensor([0, 1, indices.numel() // 2, indices.numel() - 1], device="cuda")
    want_pre = (G[rows_of[e]].double() * sae.W_dec[indices[e].long()].double()).sum(1)
    want_pre = want_pre * (values[e] > 0)
    torch.testing.assert_close(got.pre[e].double(), want_pre, atol=1e-2 * want_pre.abs().max().item(), rtol=1e-2)
    unused = torch.nonzero(counts == 0).flatten()[:3]
    if unused.numel():
        assert float(got.W_dec[unused].abs().max()) == 0 and float(got.W_enc[:, unused].abs().max()) == 0
    want_bdec = G.double().sum(0) - sae.W_enc.double() @ got.b_enc.double()
    check("b_dec", got.b_dec, want_bdec.cpu(), torch.bfloat16)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_sparse_backward_strided_layouts(dtype):
    """x as a column-major view, W_enc as the transposed view of W_dec's storage ([d_in, d_sae]
    with unit row stride), W_dec non-contiguous, dL/dx_hat in fp32 and grad_values in another
    dtype than the parameters: the same gradients as the oracle."""
    M, D, N = 200, 96, 300
    p, x, _ = make(M, D, N, "relu", dtype, seed=11, hot=2)
    Wd = p["W_dec"].cuda()
    sae = Sae(activation="relu", k=None, W_enc=Wd.t(), b_enc=p["b_enc"].cuda(),
              W_dec=Wd.t().contiguous().t(), b_dec=p["b_dec"].cuda(), threshold=None)  # W_dec column-major
    assert sae.W_enc.stride() == (1, D) and sae.W_dec.stride() == (1, N)
    xg = x.cuda().t().contiguous().t()  # column-major x
    indptr, indices, values = saeflow_amd.encode_sparse(sae, xg)
    g = torch.Generator().manual_seed(12)
    G = torch.randn(M, D, generator=g)  # fp32 upstream gradient
    H = torch.randn(indices.numel(), generator=g).to(torch.float16)
    got = sparse_backward(xg, sae.W_enc, sae.b_enc, sae.W_dec, sae.b_dec, (indptr, indices, values), G.cuda(),
                          H.cuda())
    ones = torch.ones(indices.numel(), device="cuda")
    active = (csr_to_dense(indptr, indices, ones, N).cpu() > 0) & (csr_to_dense(indptr, indices, values, N).cpu() > 0)
    Hd = csr_to_dense(indptr, indices, H.cuda().float(), N).cpu()
    # the kernels take dL/dx_hat in the parameters' dtype
    want = obwd.grads(x, Wd.t().cpu(), p["b_enc"], p["W_dec"], p["b_dec"], active, G.to(dtype), Hd)
    for name in ("W_enc", "b_enc", "W_dec", "b_dec", "x"):
        check(name, getattr(got, name), want[name], dtype)


def _layout(A, layout):
    """A [R, C] on the GPU in the given memory layout (same values)."""
    R, C = A.shape
    if layout == "rows":
        return A.cuda()
    if layout == "cols":  # unit row stride: the transpose of a contiguous [C, R]
        return A.t().contiguous().t().cuda()
    if layout == "strided":  # neither stride is 1
        big = torch.zeros(2 * R, 3 * C, dtype=A.dtype)
        big[::2, ::3] = A
        return big.cuda()[::2, ::3]
    flat = torch.zeros(R * C + 1, dtype=A.dtype)  # "offset": rows start one element past a 16-B boundary
    flat[1:] = A.reshape(-1)
    return flat.cuda()[1:].view(R, C)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("layout", ["rows", "cols", "strided", "offset"])
def test_matvec_and_column_sums_every_layout(dtype, layout):
    """sf_matvec (W v, accumulated with a sign) and sf_column_sums against float64 sums of the
    same rounded inputs, over row-major, column-major, doubly strided and misaligned operands and
    sizes that end inside a 16-B chunk, a row group or a partial range."""
    from saeflow_amd import _lib
    lib = _lib.load()
    g = torch.Generator().manual_seed(5)
    for R, C in [(1, 1), (37, 1000), (517, 20011), (64, 4096), (3, 70000)]:
        A = torch.randn(R, C, generator=g).to(dtype)
        v = torch.randn(C, generator=g)
        W = _layout(A, layout)
        assert torch.equal(W.cpu(), A)
        out0 = torch.randn(R, generator=g)
        out = out0.cuda()
        ws = torch.empty(R * min(256, C), dtype=torch.float32, device="cuda")
        _lib.check(lib.sf_matvec(_lib.ptr(W), R, C, W.stride(0), W.stride(1), _lib.DTYPE[dtype], _lib.ptr(v.cuda()),
                                 -1.0, 1, _lib.ptr(out), _lib.ptr(ws), ws.numel(), _lib.stream(W.device)))
        want = out0.double() - A.double() @ v.double()
        bound = (A.double().abs() @ v.double().abs()).max().item()
        torch.testing.assert_close(out.cpu().double(), want, atol=2e-6 * bound, rtol=0, msg=f"matvec {R}x{C}")
        if layout in ("cols", "strided"):
            continue  # sf_column_sums takes unit column stride
        sums = torch.empty(C, dtype=torch.float32, device="cuda")
        ws = torch.empty(min(256, R) * C, dtype=torch.float32, device="cuda")
        _lib.check(lib.sf_column_sums(_lib.ptr(W), R, C, W.stride(0), _lib.DTYPE[dtype], 2.0, 0, _lib.ptr(sums),
                                      _lib.ptr(ws), ws.numel(), _lib.stream(W.device)))
        want = 2.0 * A.double().sum(0)
        bound = A.double().abs().sum(0).max().item()
        torch.testing.assert_close(sums.cpu().double(), want, atol=4e-6 * bound, rtol=0, msg=f"column sums {R}x{C}")


@pytest.mark.parametrize("dtype,D,N", [(torch.bfloat16, 1088, 200), (torch.float32, 520, 136),
                                       (torch.float16, 1088, 203)])
def test_sparse_backward_feature_lengths_around_the_thresholds(dtype, D, N):
    """Features of exactly 0, 1, 63, 64, 65, 255, 256, 257, 300 and 513 entries: up to 64 entries
    a feature's dW_enc column is summed in the LDS tile, above that from fp32 partial slots, and
    above 256 from several work items. D spans full 512-element (fp32: 256) slabs and a partial
    one; N leaves a partial 64-feature tile, and N = 203 makes the dW_enc rows unaligned (the
    element-store path). The CSR is built directly, with values = the forward's pre > 0."""
    M = 600
    rng = np.random.default_rng(7)
    lengths = [0, 1, 2, 63, 64, 65, 66, 255, 256, 257, 300, 513]
    lengths += list(rng.integers(0, 6, N - len(lengths)))
    order = rng.permutation(N)  # spread the long features over the tiles
    mask = np.zeros((M, N), dtype=bool)
    for j, n in zip(order, lengths):
        mask[rng.choice(M, size=n, replace=False), j] = True
    g = torch.Generator().manual_seed(3)
    W_dec = torch.randn(N, D, generator=g) / D ** 0.5
    W_enc = torch.randn(D, N, generator=g) / D ** 0.5
    b_enc = torch.full((N,), 4.0)  # pre > 0 on every stored entry
    b_dec = torch.randn(D, generator=g) * 0.1
    x = torch.randn(M, D, generator=g)
    W_dec, W_enc, b_enc, b_dec, x = (t.to(dtype) for t in (W_dec, W_enc, b_enc, b_dec, x))
    pre = (x.double() - b_dec.double()) @ W_enc.double() + b_enc.double()
    rows, cols = np.nonzero(mask)  # row-major: a canonical CSR
    indptr = torch.from_numpy(np.concatenate([[0], np.cumsum(mask.sum(1))]).astype(np.int64))
    indices = torch.from_numpy(cols.astype(np.int32))
    values = pre[torch.from_numpy(rows), torch.from_numpy(cols)].to(dtype)
    assert float(values.double().min()) > 0
    G = torch.randn(M, D, generator=g).to(dtype)
    H = torch.randn(len(rows), generator=g).to(dtype)
    got = sparse_backward(x.cuda(), W_enc.cuda(), b_enc.cuda(), W_dec.cuda(), b_dec.cuda(),
                          (indptr.cuda(), indices.cuda(), values.cuda()), G.cuda(), H.cuda())
    Hd = torch.zeros(M, N, dtype=torch.float64)
    Hd[torch.from_numpy(rows), torch.from_numpy(cols)] = H.double()
    want = obwd.grads(x, W_enc, b_enc, W_dec, b_dec, torch.from_numpy(mask), G, Hd)
    for name in ("W_enc", "b_enc", "W_dec", "b_dec", "x"):
        check(name, getattr(got, name), want[name], dtype)
    # unused features: exactly zero gradients
    unused = torch.from_numpy(~mask.any(0))
    assert int(unused.sum()) > 0
    assert torch.count_nonzero(got.W_enc.cpu()[:, unused]) == 0 and torch.count_nonzero(got.W_dec.cpu()[unused]) == 0
    assert torch.count_nonzero(got.b_enc.cpu()[unused]) == 0
