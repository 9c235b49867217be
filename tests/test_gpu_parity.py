"""GPU parity: the gfx950 kernels, called through the C ABI, against the CPU oracle.

Mirrors the reference's tests/test_kernels.py (shapes, dtypes, parameter recipe, tolerance
and near-cut exclusion, exact row counts, bit-exact CSR) and adds the vector-path shapes,
the committed golden fixtures, and size-independent properties at the benchmark sizes.

Tolerances: fp32 rtol 1e-5 (atol 1e-5 * (1 + max|pre|)), bf16 rtol 2e-2, fp16 rtol 5e-3,
each with atol = rtol * (1 + max|pre|) against the fp32/fp64 oracle computed from the same
rounded inputs; elements within atol of the ReLU / JumpReLU cut are excluded; CSR indptr
and indices and the copied values are compared bit-exactly.
"""

import random
from pathlib import Path

import numpy as np
import pytest
import torch

import saeflow_amd
from oracle import csr as ocsr
from oracle import reference as oref
from saeflow_amd import workloads
from saeflow_amd.kernels import (best_config, csr_to_dense, dense_to_csr, encode_pre, encode_rows, fused_encode,
                                 sparse_decode, topk_rows)

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
SHAPES = [(1, 16, 32), (37, 50, 129), (64, 64, 256), (100, 33, 70)]  # reference test_kernels.py:9
VEC_SHAPES = [(300, 128, 520), (257, 64, 264), (16, 2304, 512)]     # 16-B paths, ragged M / N tiles
DTYPES = [torch.float32, torch.bfloat16, torch.float16]
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 5e-3}


def make_params(d_in, d_sae, activation, dtype, seed=0, k=None):
    """Reference make_sae recipe (test_kernels.py:14-20) on CPU with an explicit generator."""
    g = torch.Generator().manual_seed(seed)
    W_dec = torch.randn(d_sae, d_in, generator=g)
    W_dec /= W_dec.norm(dim=1, keepdim=True)
    p = dict(W_dec=W_dec, W_enc=W_dec.T.contiguous(), b_enc=torch.randn(d_sae, generator=g) * 0.1,
             b_dec=torch.randn(d_in, generator=g) * 0.1,
             threshold=torch.rand(d_sae, generator=g) * 0.5 if activation == "jumprelu" else None)
    return {k_: (v.to(dtype) if v is not None else None) for k_, v in p.items()}


def gpu(p):
    return {k: (v.cuda() if torch.is_tensor(v) else v) for k, v in p.items()}


class Sae:
    def __init__(self, p, activation, k=None):
        self.__dict__.update(p)
        self.activation, self.k = activation, k


def check_encode(got, x, p, activation, dtype):
    """Reference recipe (test_kernels.py:33-44) with the stated tolerance."""
    pre = oref.encode_pre(x, p["W_enc"], p["b_enc"], p["b_dec"], dtype=torch.float64)
    want = oref.activate(pre, activation, p["threshold"])
    cut = pre - (p["threshold"].double() if activation == "jumprelu" else 0)
    tol = TOL[dtype] * (1 + pre.abs().max())
    keep = cut.abs() > tol
    torch.testing.assert_close(got.cpu().double()[keep], want[keep], atol=float(tol), rtol=TOL[dtype])


# ----------------------------------------------------------------------------- encode


def tilings(dtype):
    bk = 32 if dtype == torch.float32 else 64
    return [None, {"BLOCK_M": 256, "BLOCK_N": 128, "BLOCK_K": bk // 2, "GROUP_M": 2},
            {"BLOCK_M": 256, "BLOCK_N": 256, "BLOCK_K": bk, "GROUP_M": 1, "NUM_WAVES": 4}]


@pytest.mark.parametrize("narrow", [0, 1, 2])
@pytest.mark.parametrize("activation", ["relu", "jumprelu"])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", SHAPES + VEC_SHAPES)
def test_fused_encode(shape, dtype, activation, narrow):
    M, d_in, d_sae = shape
    p = make_params(d_in, d_sae, activation, dtype)
    x = torch.randn(M, d_in).to(dtype)
    q = gpu(p)
    row_nnz = torch.zeros(M, device="cuda", dtype=torch.int32)
    got = fused_encode(x.cuda(), q["W_enc"], q["b_enc"], q["b_dec"], q["threshold"], activation, row_nnz=row_nnz,
                       config=tilings(dtype)[narrow])
    assert got.dtype == dtype and got.shape == (M, d_sae)
    check_encode(got, x, p, activation, dtype)
    # counts are of the stored values (test_kernels.py:44)
    assert torch.equal(row_nnz.cpu(), torch.count_nonzero(got, dim=1).int().cpu())


@pytest.mark.parametrize("whole", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_tile_orders_cover_every_tile_once(dtype, whole):
    # 6 x 9 tiles of 256x256 (6 x 17 of 256x128): ragged runs of token tiles (GROUP_M) and of
    # feature tiles (GROUP_N), groups wider than the grid included. With b_enc = 10 every
    # relu output is kept, so a tile skipped or computed twice shows in the row counts; the
    # features are bit-identical in every order. Whole tiles (1536 x 2304) run the 8-wave
    # orders through the persistent kernel.
    M, d_in, d_sae = (1536, 64, 2304) if whole else (1300, 64, 2100)
    p = make_params(d_in, d_sae, "relu", dtype)
    x = torch.randn(M, d_in).to(dtype).cuda()
    q = gpu(p)
    b_enc = torch.full_like(q["b_enc"], 10.0)
    bk = 32 if dtype == torch.float32 else 64
    orders = [(1, 1), (1, 2), (1, 4), (1, 8), (1, 100), (2, 0), (4, 0), (5, 0), (100, 0)]
    cfgs = [{"BLOCK_M": 256, "BLOCK_N": 256, "BLOCK_K": bk, "GROUP_M": gm, "NUM_WAVES": w, "GROUP_N": gn}
            for w in (8, 4) for gm, gn in orders]
    cfgs += [{"BLOCK_M": 256, "BLOCK_N": 128, "BLOCK_K": bk // 2, "GROUP_M": gm, "NUM_WAVES": 4, "GROUP_N": gn}
             for gm, gn in [(1, 3), (1, 8), (3, 0)]]
    bits = torch.int32 if dtype == torch.float32 else torch.int16
    want = None
    for cfg in [None] + cfgs:
        row_nnz = torch.zeros(M, device="cuda", dtype=torch.int32)
        got = fused_encode(x, q["W_enc"], b_enc, q["b_dec"], None, "relu", row_nnz=row_nnz, config=cfg)
        assert torch.all(row_nnz == d_sae), cfg
        if want is None:
            want = got
            check_encode(got, x.cpu(), {**p, "b_enc": b_enc.cpu()}, "relu", dtype)
        else:
            assert torch.equal(got.view(bits), want.view(bits)), cfg
    # the row-candidate kernels take the same orders
    for cfg in cfgs[:9]:
        cnt, idx, val = encode_rows(x, q["W_enc"], b_enc, q["b_dec"], None, "relu", cap=16, config=cfg)
        assert torch.all(cnt == d_sae), cfg


@pytest.mark.parametrize("waves", [8, 4])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("kmajor", [False, True])
@pytest.mark.parametrize("shape", [(256, 64, 256), (512, 96, 768), (1536, 192, 2304), (4096, 320, 8448)])
def test_persistent_encode_equals_one_tile_per_workgroup(shape, kmajor, dtype, waves):
    """Whole-tile shapes (M and d_sae multiples of 256) run the persistent form of the 256x256
    kernel (8 waves of 128x64 or 4 of 128x128): one workgroup per CU walking its XCD's tiles,
    the next tile's loads under the epilogue. One more token row makes the same problem ragged,
    which runs one workgroup per tile: the first M rows agree bit for bit, row counts included,
    for both activations, both W layouts and fp32 output. One tile and 2 x 3 tiles leave XCDs
    with no tile (their workgroups exit at once); the larger shape (16 x 33 tiles) gives
    workgroups two or three tiles of both buffer parities."""
    M, d_in, d_sae = shape
    bits = {torch.float32: torch.int32, torch.bfloat16: torch.int16, torch.float16: torch.int16}
    bk = 32 if dtype == torch.float32 else 64
    cfg = {"BLOCK_M": 256, "BLOCK_N": 256, "BLOCK_K": bk, "GROUP_M": 1, "NUM_WAVES": waves, "GROUP_N": 8}
    for activation in ("relu", "jumprelu"):
        p = make_params(d_in, d_sae, activation, dtype)
        q = gpu(p)
        W = q["W_enc"].T.contiguous().T if kmajor else q["W_enc"]
        x = torch.randn(M + 1, d_in).to(dtype).cuda()
        for out_dtype in [None] + ([torch.float32] if dtype != torch.float32 else []):
            rn_p = torch.zeros(M, device="cuda", dtype=torch.int32)
            rn_t = torch.zeros(M + 1, device="cuda", dtype=torch.int32)
            got_p = fused_encode(x[:M], W, q["b_enc"], q["b_dec"], q["threshold"], activation, row_nnz=rn_p,
                                 out_dtype=out_dtype, config=cfg)
            got_t = fused_encode(x, W, q["b_enc"], q["b_dec"], q["threshold"], activation, row_nnz=rn_t,
                                 out_dtype=out_dtype, config=cfg)
            b = bits[got_p.dtype]
            assert torch.equal(got_p.view(b), got_t[:M].view(b)), (activation, out_dtype)
            assert torch.equal(rn_p, rn_t[:M]), (activation, out_dtype)
            if out_dtype is None and not kmajor:
                check_encode(got_p, x[:M].cpu(), p, activation, dtype)


def test_persistent_encode_random_whole_tile_problems():
    """Seeded random whole-tile problems (tokens and features multiples of 256, any d_in) over
    both W layouts, both wave counts, both tile orders with their group widths, both
    activations and fp32 output: the persistent kernel on M rows equals one workgroup per tile
    on M + 1 rows bit for bit, row counts included."""
    rng = random.Random(1234)
    for case in range(30):
        dtype = rng.choice(DTYPES)
        M, N = 256 * rng.randint(1, 8), 256 * rng.randint(1, 24)
        K = rng.choice([16, 100, 192, 500, 768, 1000])
        bk = 32 if dtype == torch.float32 else 64
        cfg = {"BLOCK_M": 256, "BLOCK_N": 256, "BLOCK_K": bk, "GROUP_M": rng.choice([1, 2, 4]),
               "NUM_WAVES": rng.choice([8, 4]), "GROUP_N": rng.choice([0, 1, 3, 8, 16])}
        act = rng.choice(["relu", "jumprelu"])
        g = torch.Generator().manual_seed(case)
        W = (torch.randn(K, N, generator=g) / K ** 0.5).to(dtype).cuda()
        if rng.random() < 0.3:
            W = W.t().contiguous().t()
        b_enc = (torch.randn(N, generator=g) * 0.1 - 0.2).to(dtype).cuda()
        b_dec = (torch.randn(K, generator=g) * 0.1).to(dtype).cuda()
        thr = (torch.rand(N, generator=g) * 0.5).to(dtype).cuda() if act == "jumprelu" else None
        x = torch.randn(M + 1, K, generator=g).to(dtype).cuda()
        for od in [None] + ([torch.float32] if dtype != torch.float32 else []):
            rp = torch.zeros(M, device="cuda", dtype=torch.int32)
            rt = torch.zeros(M + 1, device="cuda", dtype=torch.int32)
            got = fused_encode(x[:M], W, b_enc, b_dec, thr, act, row_nnz=rp, out_dtype=od, config=cfg)
            want = fused_encode(x, W, b_enc, b_dec, thr, act, row_nnz=rt, out_dtype=od, config=cfg)
            bits = torch.int32 if got.dtype == torch.float32 else torch.int16
            assert torch.equal(got.view(bits), want[:M].view(bits)), (case, dtype, M, N, K, cfg, act, od)
            assert torch.equal(rp, rt[:M]), (case, dtype, M, N, K, cfg, act, od)


@pytest.mark.parametrize("dtype", DTYPES)
def test_fused_encode_strided_weights(dtype):
    # column-major W_enc (test_kernels.py:47-52): the K-contiguous MFMA path
    p = make_params(48, 80, "relu", dtype)
    x = torch.randn(20, 48).to(dtype)
    q = gpu(p)
    W_t = q["W_enc"].T.contiguous().T
    got = fused_encode(x.cuda(), W_t, q["b_enc"], q["b_dec"])
    check_encode(got, x, p, "relu", dtype)
    # arbitrary (non-unit) strides: generic path
    W_s = torch.empty(48, 160, device="cuda", dtype=dtype)[:, ::2]
    W_s.copy_(q["W_enc"])
    got = fused_encode(x.cuda(), W_s, q["b_enc"], q["b_dec"])
    check_encode(got, x, p, "relu", dtype)


def test_fused_encode_mixed_dtypes_and_out_dtype():
    # x fp32 with bf16 weights: x' is formed in fp32 and rounded to bf16 (encode.py:72)
    p = make_params(64, 256, "relu", torch.bfloat16)
    x = torch.randn(33, 64)
    q = gpu(p)
    got = fused_encode(x.cuda(), q["W_enc"], q["b_enc"], q["b_dec"], out_dtype=torch.float32)
    assert got.dtype == torch.float32
    check_encode(got, x, p, "relu", torch.bfloat16)


def test_encode_pre_and_config():
    p = make_params(64, 256, "relu", torch.float32)
    x = torch.randn(40, 64)
    q = gpu(p)
    got = encode_pre(x.cuda(), q["W_enc"], q["b_enc"], q["b_dec"])  # small: the default tiling
    want = oref.encode_pre(x, p["W_enc"], p["b_enc"], p["b_dec"], dtype=torch.float64)
    torch.testing.assert_close(got.cpu().double(), want, atol=1e-5 * (1 + want.abs().max().item()), rtol=1e-5)
    cfg = best_config()
    assert cfg == {"BLOCK_M": 256, "BLOCK_N": 256, "BLOCK_K": 32, "GROUP_M": 1, "NUM_WAVES": 8, "GROUP_N": 8}
    got2 = fused_encode(x.cuda(), q["W_enc"], q["b_enc"], q["b_dec"], config={**cfg, "GROUP_M": 3, "GROUP_N": 0})
    torch.testing.assert_close(got2, torch.relu(got))
    narrow = {"BLOCK_M": 256, "BLOCK_N": 128, "BLOCK_K": 16, "GROUP_M": 2}
    got3 = fused_encode(x.cuda(), q["W_enc"], q["b_enc"], q["b_dec"], config=narrow)
    torch.testing.assert_close(got3, torch.relu(got), atol=1e-5, rtol=1e-5)
    assert best_config() == cfg  # pinned configs are not tuning results (encode.py:142-144)
    with pytest.raises(ValueError, match="tile config"):
        fused_encode(x.cuda(), q["W_enc"], q["b_enc"], q["b_dec"], config={"BLOCK_M": 64})


def test_autotune_picks_a_compiled_tiling_with_identical_results():
    from saeflow_amd.kernels import encode as kenc
    sae, x, meta = workloads.make("C2", T=4096, device="cuda")
    assert 2 * 4096 * 2304 * 16384 >= kenc.AUTOTUNE_MIN_FLOPS
    kenc._tuned.clear()
    prior = torch.arange(4096, device="cuda", dtype=torch.int32)
    row_nnz = prior.clone()  # counts accumulate into what the caller passed, tuning or not
    f = fused_encode(x, sae.W_enc, sae.b_enc, sae.b_dec, sae.threshold, "jumprelu", row_nnz=row_nnz)
    assert len(kenc._tuned) == 1 and best_config() in kenc._candidates(torch.bfloat16)
    want_cnt = torch.count_nonzero(f, dim=1).int()
    assert torch.equal(row_nnz - prior, want_cnt)
    for cfg in kenc._candidates(torch.bfloat16):
        g = fused_encode(x, sae.W_enc, sae.b_enc, sae.b_dec, sae.threshold, "jumprelu", config=cfg)
        assert torch.equal(g, f)


@pytest.mark.parametrize("name,dtype", [("C1", None), ("C2", None), ("C2", torch.float16)])
def test_every_tiling_is_repeatable_and_identical(name, dtype):
    # Every tiling accumulates each output in the same K order, so results must agree bit for
    # bit across tilings and across repeated launches. Sized so every kernel runs several
    # hundred workgroups over many K-steps: a pipeline race (a stage overwritten while
    # another wave still reads it) shows up as rare differing tiles.
    from saeflow_amd.kernels import encode as kenc
    sae, x, meta = workloads.make(name, T=2048, dtype=dtype, device="cuda")
    M = x.shape[0]
    ref = None
    for cfg in kenc._candidates(sae.W_enc.dtype):
        for _ in range(3):
            row_nnz = torch.zeros(M, device="cuda", dtype=torch.int32)
            f = fused_encode(x, sae.W_enc, sae.b_enc, sae.b_dec, sae.threshold, sae.activation, row_nnz=row_nnz,
                             config=cfg)
            if ref is None:
                ref = (f, row_nnz)
                assert torch.equal(row_nnz, torch.count_nonzero(f, dim=1).int())
            assert torch.equal(f, ref[0]) and torch.equal(row_nnz, ref[1]), cfg


@pytest.mark.parametrize("name", ["encode_relu", "encode_jumprelu", "encode_relu_bf16"])
def test_fused_encode_golden(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        g = {k: z[k] for k in z.files}
    act = str(g["activation"])
    dtype = torch.bfloat16 if bool(g["bf16"]) else torch.float32
    T = lambda a: torch.from_numpy(a).to(dtype).cuda()  # noqa: E731  (exact: values are representable)
    got = fused_encode(T(g["x"]), T(g["W_enc"]), T(g["b_enc"]), T(g["b_dec"]), T(g["threshold"]), act,
                       out_dtype=torch.float32)
    pre = torch.from_numpy(g["pre"])
    tol = (1e-5 if dtype == torch.float32 else 2e-2) * (1 + pre.abs().max().item())
    cut = pre - (torch.from_numpy(g["threshold"]).double() if act == "jumprelu" else 0)
    keep = cut.abs() > tol
    torch.testing.assert_close(got.cpu().double()[keep], torch.from_numpy(g["out"])[keep], atol=tol, rtol=1e-5)


# ----------------------------------------------------------------------------- dense -> CSR


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(1, 32), (37, 129), (64, 300), (5, 4096), (3, 1000), (1, 5), (3, 20003),
                                   (4, 70001)])
def test_dense_to_csr_matches_torch(shape, dtype):
    f = torch.relu(torch.randn(*shape) - 1.0).to(dtype)
    f[0] = 0  # an empty row
    bits = torch.int32 if dtype == torch.float32 else torch.int16
    for row_nnz in (None, torch.count_nonzero(f, dim=1).int()):
        indptr, indices, values = dense_to_csr(f.cuda(), None if row_nnz is None else row_nnz.cuda())
        want = f.to_sparse_csr()
        assert torch.equal(indptr.cpu(), want.crow_indices())
        assert torch.equal(indices.long().cpu(), want.col_indices())
        assert torch.equal(values.cpu().view(bits), want.values().view(bits))


@pytest.mark.parametrize("dtype", DTYPES)
def test_dense_to_csr_rows_of_a_megabyte_and_more(dtype):
    # rows of >= 1 MiB take the 16-wave shape: staged rows (few nonzeros), a row longer than the
    # staging (direct stores), an empty row and a ragged tail of columns
    N = (1 << 20) // torch.tensor([], dtype=dtype).element_size() + 3
    f = torch.zeros(5, N, dtype=dtype)
    g = torch.Generator().manual_seed(5)
    for r, n in ((0, 100), (1, 3000), (3, 1), (4, 2048)):
        cols = torch.randperm(N, generator=g)[:n]
        f[r, cols] = (torch.rand(n, generator=g) + 0.25).to(dtype)
    f[4, N - 2:] = 1.0  # nonzeros in the tail columns
    bits = torch.int32 if dtype == torch.float32 else torch.int16
    indptr, indices, values = dense_to_csr(f.cuda())
    want = f.to_sparse_csr()
    assert torch.equal(indptr.cpu(), want.crow_indices())
    assert torch.equal(indices.long().cpu(), want.col_indices())
    assert torch.equal(values.cpu().view(bits), want.values().view(bits))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_compact_keeps_to_the_announced_segments(dtype):
    """Counts that understate or overstate a row only change that row's segment: an
    understated row gets its first nonzeros in column order, an overstated row's extra
    slots are left as they were, and nothing is written outside [indptr[m], indptr[m+1])."""
    f = torch.relu(torch.randn(6, 20003) - 1.0).to(dtype)  # rows span several load groups
    true = torch.count_nonzero(f, dim=1).int()
    counts = true.clone()
    counts[1] -= 5
    counts[3] += 7
    indptr = torch.zeros(7, dtype=torch.int64)
    indptr[1:] = torch.cumsum(counts.long(), 0)
    nnz = int(indptr[-1])
    sentinel = -12345
    indices = torch.full((nnz,), sentinel, dtype=torch.int32, device="cuda")
    values = torch.zeros(nnz, dtype=dtype, device="cuda")
    from saeflow_amd import _lib
    fg, ig = f.cuda(), indptr.cuda()
    _lib.check(_lib.load().sf_compact(_lib.ptr(fg), fg.stride(0), fg.stride(1), _lib.dtype_code(fg, "f"), 6,
                                      fg.shape[1], _lib.ptr(ig), nnz, _lib.ptr(indices), _lib.ptr(values),
                                      _lib.stream(fg.device)))
    got = indices.cpu()
    for m in range(6):
        cols = torch.nonzero(f[m]).flatten().int()
        seg = got[indptr[m]:indptr[m + 1]]
        k = min(int(counts[m]), int(true[m]))
        assert torch.equal(seg[:k], cols[:k])
        assert bool((seg[k:] == sentinel).all())


@pytest.mark.parametrize("dtype", DTYPES)
def test_dense_to_csr_special_values(dtype):
    """-0.0 is a zero; NaN, +-inf and subnormals are nonzeros (torch's `x != 0`), in rows that
    span several load groups and end in a ragged tail."""
    g = torch.Generator().manual_seed(3)
    f = torch.zeros(3, 20003)
    specials = torch.tensor([-0.0, float("nan"), float("inf"), -float("inf"), 1e-40, 6e-8, -2.5])
    idx = torch.randint(0, f.numel(), (400,), generator=g)
    f.view(-1)[idx] = specials[torch.randint(0, len(specials), (400,), generator=g)]
    f[1, -3:] = torch.tensor([float("nan"), -0.0, 1.0])  # the tail past the last whole chunk
    f = f.to(dtype)
    bits = torch.int32 if dtype == torch.float32 else torch.int16
    for row_nnz in (None, torch.count_nonzero(f, dim=1).int()):
        indptr, indices, values = dense_to_csr(f.cuda(), None if row_nnz is None else row_nnz.cuda())
        want = f.to_sparse_csr()
        assert torch.equal(indptr.cpu(), want.crow_indices())
        assert torch.equal(indices.long().cpu(), want.col_indices())
        assert torch.equal(values.cpu().view(bits), want.values().view(bits))


def test_dense_to_csr_all_zero():
    indptr, indices, values = dense_to_csr(torch.zeros(5, 40, device="cuda"))
    assert indptr.tolist() == [0] * 6 and indices.numel() == 0 and values.numel() == 0


def test_dense_to_csr_golden_and_strided():
    with np.load(GOLDEN / "csr.npz", allow_pickle=False) as z:
        g = {k: z[k] for k in z.files}
    f = torch.from_numpy(g["f"]).cuda()
    for src in (f, f.T.contiguous().T, f.to(torch.bfloat16)):
        indptr, indices, values = dense_to_csr(src)
        assert indptr.cpu().numpy().tolist() == g["indptr"].tolist()
        assert indices.cpu().numpy().tolist() == g["indices"].tolist()
        want = torch.from_numpy(g["values"]).to(src.dtype).float().numpy()
        np.testing.assert_array_equal(values.float().cpu().numpy(), want)


# ----------------------------------------------------------------------------- decode


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", SHAPES + [(64, 2304, 4096), (9, 4096, 1000), (5, 6000, 300)])
def test_sparse_decode(shape, dtype):
    M, d_in, d_sae = shape
    p = make_params(d_in, d_sae, "relu", dtype)
    f = torch.relu(torch.randn(M, d_sae) - 1.5).to(dtype)  # ~7% density, variable L0
    q = gpu(p)
    got = sparse_decode(*dense_to_csr(f.cuda()), q["W_dec"], q["b_dec"]).cpu().double()
    want = f.double() @ p["W_dec"].double() + p["b_dec"].double()
    # test_kernels.py:76-79 recipe against an fp64 dense product
    torch.testing.assert_close(got, want, atol=4 * TOL[dtype], rtol=TOL[dtype])


def test_sparse_decode_golden_and_options():
    with np.load(GOLDEN / "decode.npz", allow_pickle=False) as z:
        g = {k: z[k] for k in z.files}
    W = torch.from_numpy(g["W_dec"]).cuda()
    b = torch.from_numpy(g["b_dec"]).cuda()
    csr = tuple(torch.from_numpy(g[k]).cuda() for k in ("indptr", "indices", "values"))
    want = torch.from_numpy(g["out"])
    got = sparse_decode(*csr, W, b).cpu().double()
    torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-5)
    assert got[1].sub(torch.from_numpy(g["b_dec"]).double()).abs().max() < 1e-7  # empty row = b_dec
    nob = sparse_decode(*csr, W).cpu().double()
    torch.testing.assert_close(nob, want - torch.from_numpy(g["b_dec"]).double(), atol=1e-5, rtol=1e-5)
    # strided W_dec (generic path), int64 indices, bf16 output
    Ws = W.T.contiguous().T
    torch.testing.assert_close(sparse_decode(csr[0], csr[1].long(), csr[2], Ws, b).cpu().double(), want,
                               atol=1e-5, rtol=1e-5)
    out16 = sparse_decode(*csr, W, b, out_dtype=torch.bfloat16)
    assert out16.dtype == torch.bfloat16
    torch.testing.assert_close(out16.cpu().double(), want, atol=2e-2, rtol=2e-2)
    # out-of-range indices contribute nothing
    bad = csr[1].clone()
    bad[0] = 10_000
    got_bad = sparse_decode(csr[0], bad, csr[2], W, b).cpu().double()
    fix = csr[2].clone()
    fix[0] = 0
    torch.testing.assert_close(got_bad, sparse_decode(csr[0], csr[1], fix, W, b).cpu().double())


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("M,d_in,d_sae", [(77, 2304, 3000), (33, 64, 500), (5, 192, 70), (260, 512, 9000),
                                         (40, 4160, 300)])
def test_line_slab_decode_matches_row_decode(M, d_in, d_sae, dtype):
    """Rows of whole 128-B lines take the line-slab kernel (slab-major units split over the
    XCDs; slabs of two lines, one token per 16 lanes and 64 pairs per batch, where the row has
    an even number of lines and d_sae <= 65536, else one line, 8 lanes, 32 pairs); config=
    forces the one-row-per-wavefront kernel. Both sum each output over its entries in CSR
    order, so they agree bit for bit: here with empty rows, rows longer than one batch (300 and
    1000 pairs), invalid indices (-1, d_sae) and M not a multiple of a workgroup's 16 or 32
    tokens. Both slab widths appear (bf16 d_in 64, 192 and 4160 have an odd number of lines).
    d_in = 4160 in fp32 makes a 16640-B row pitch, past a buffer record's 14-bit stride: the
    line-slab kernel's 64-bit-load form (16-bit types keep the buffer form at 8320 B)."""
    g = torch.Generator().manual_seed(M + d_in)
    p = make_params(d_in, d_sae, "relu", dtype)
    lens = torch.randint(0, 120, (M,), generator=g)
    lens[0] = 0
    lens[min(3, M - 1)] = 300
    lens[M // 2] = 1000
    lens[M - 1] = 0
    indptr = torch.zeros(M + 1, dtype=torch.int64)
    indptr[1:] = torch.cumsum(lens, 0)
    nnz = int(indptr[-1])
    indices = torch.randint(0, d_sae, (nnz,), generator=g, dtype=torch.int32)
    indices[::97] = -1
    indices[5::131] = d_sae
    values = torch.randn(nnz, generator=g).to(dtype)
    W, b = p["W_dec"].cuda(), p["b_dec"].cuda()
    csr = (indptr.cuda(), indices.cuda(), values.cuda())
    got = sparse_decode(*csr, W, b)
    want = sparse_decode(*csr, W, b, config={"BLOCK_NNZ": 64, "BLOCK_D": 1 << 20})
    assert torch.equal(got, want)
    for out_dtype in (torch.float32, torch.bfloat16):  # 16-B stores and element-wise stores
        got_o = sparse_decode(*csr, W, b, out_dtype=out_dtype)
        assert torch.equal(got_o, sparse_decode(*csr, W, b, out_dtype=out_dtype,
                                                config={"BLOCK_NNZ": 64, "BLOCK_D": 1 << 20}))
    ok = (indices >= 0) & (indices < d_sae)
    ref = ocsr.sparse_decode(indptr.numpy(), np.where(ok, indices, 0).astype(np.int32),
                             np.where(ok, values.double().numpy(), 0.0), p["W_dec"].double().numpy(),
                             p["b_dec"].double().numpy())
    torch.testing.assert_close(got.cpu().double(), torch.from_numpy(ref), atol=8 * TOL[dtype], rtol=TOL[dtype])


@pytest.mark.parametrize("dtype,d_in", [(torch.bfloat16, 512), (torch.float32, 4160)])
def test_line_slab_decode_padding_never_reads_feature_zero(dtype, d_in):
    """Padding pairs (a wavefront walks its longest token's entries; a round of U rows its
    last spare pairs) and invalid indices must add nothing whatever W_dec holds, as the
    reference's masked load gives (decode.py:46-50): with NaN and Inf in W_dec row 0 and no
    token using feature 0, every output is finite, in all three kernels. bf16 d_in 512 takes
    the buffer-resource gathers (a record index past d_sae reads zeros), fp32 d_in 4160 (a
    16640-B pitch) the 64-bit loads (a padding pair skips its load)."""
    M, d_sae = 96, 700
    g = torch.Generator().manual_seed(d_in)
    p = make_params(d_in, d_sae, "relu", dtype)
    W = p["W_dec"].clone()
    W[0, ::2] = float("nan")
    W[0, 1::2] = float("inf")
    lens = torch.randint(1, 150, (M,), generator=g)
    lens[5] = 400  # one long token per wavefront group of 8 at least
    indptr = torch.zeros(M + 1, dtype=torch.int64)
    indptr[1:] = torch.cumsum(lens, 0)
    nnz = int(indptr[-1])
    indices = torch.randint(1, d_sae, (nnz,), generator=g, dtype=torch.int32)
    indices[::37] = -1  # invalid: also row 0's stand-in must not be read
    values = torch.randn(nnz, generator=g).to(dtype)
    csr = (indptr.cuda(), indices.cuda(), values.cuda())
    got = sparse_decode(*csr, W.cuda(), p["b_dec"].cuda())
    assert bool(torch.isfinite(got).all())
    # the row kernel (rounds of U rows: the last round's spare pairs) and the element-wise
    # kernel of strided W_dec (invalid indices) agree, finite too
    assert torch.equal(got, sparse_decode(*csr, W.cuda(), p["b_dec"].cuda(),
                                          config={"BLOCK_NNZ": 64, "BLOCK_D": 1 << 20}))
    Ws = torch.empty(d_sae, 2 * d_in, device="cuda", dtype=dtype)[:, ::2]
    Ws.copy_(W.cuda())
    assert torch.equal(got, sparse_decode(*csr, Ws, p["b_dec"].cuda()))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_decode_of_aliased_w_dec_rows(dtype):
    """W_dec views whose rows alias each other: every row the same storage (expand, row stride
    0) and rows overlapping by all but 16 B (as_strided). Both have 16-B aligned contiguous rows
    of whole 128-B lines, so they take the line-slab kernel, whose structured buffer then has a
    record stride of 0 or 16 B, below the 128-B slab its lanes read: the hardware still bounds
    the record index (not the byte offset) and reads every lane's chunk. Checked against the
    oracle on the materialized W_dec and against the contiguous copy, bit for bit."""
    M, d_in, d_sae = 40, 256, 100
    g = torch.Generator().manual_seed(7)
    one = torch.randn(1, d_in, generator=g).to(dtype)
    flat = torch.randn(d_sae * 8 + d_in, generator=g).to(dtype)
    es = 4 if dtype == torch.float32 else 2
    lens = torch.randint(0, 40, (M,), generator=g)
    indptr = torch.zeros(M + 1, dtype=torch.int64)
    indptr[1:] = torch.cumsum(lens, 0)
    nnz = int(indptr[-1])
    indices = torch.randint(0, d_sae, (nnz,), generator=g, dtype=torch.int32)
    values = torch.randn(nnz, generator=g).to(dtype)
    b = torch.randn(d_in, generator=g).to(dtype)
    csr = (indptr.cuda(), indices.cuda(), values.cuda())
    for W in (one.cuda().expand(d_sae, d_in), flat.cuda().as_strided((d_sae, d_in), (16 // es, 1))):
        got = sparse_decode(*csr, W, b.cuda()).cpu().double()
        want = ocsr.sparse_decode(indptr.numpy(), indices.numpy(), values.double().numpy(),
                                  W.cpu().double().numpy(), b.double().numpy())
        torch.testing.assert_close(got, torch.from_numpy(want), atol=8 * TOL[dtype], rtol=TOL[dtype])
        assert torch.equal(sparse_decode(*csr, W.contiguous(), b.cuda()).cpu().double(), got)


@pytest.mark.parametrize("d_sae", [460_000, 470_000])
def test_line_slab_decode_across_the_2gib_buffer_limit(d_sae):
    """W_dec of d_sae x 2304 bf16 just under 2^31 bytes (2.12 GB: rows read through a
    structured buffer resource, whose row * stride offset is 32-bit) and just over it
    (2.17 GB: 64-bit addressed loads). 80% of the gathered rows sit in the top 40000 rows,
    past 2^31 / 4608 B for the larger W_dec, where a wrapped offset would read another row:
    the line-slab kernel agrees bit for bit with the row kernel (64-bit addresses throughout),
    and sampled rows with the oracle."""
    D = 2304
    assert (d_sae * D * 2 < 2 ** 31) == (d_sae == 460_000)
    gd = torch.Generator(device="cuda").manual_seed(d_sae)
    W = torch.randn(d_sae, D, device="cuda", generator=gd).to(torch.bfloat16)
    b = torch.randn(D, device="cuda", generator=gd).to(torch.bfloat16)
    g = torch.Generator().manual_seed(d_sae + 1)
    M = 200
    lens = torch.randint(1, 90, (M,), generator=g)
    indptr = torch.zeros(M + 1, dtype=torch.int64)
    indptr[1:] = torch.cumsum(lens, 0)
    nnz = int(indptr[-1])
    top = torch.randint(d_sae - 40_000, d_sae, (nnz,), generator=g, dtype=torch.int32)
    anywhere = torch.randint(0, d_sae, (nnz,), generator=g, dtype=torch.int32)
    indices = torch.where(torch.rand(nnz, generator=g) < 0.8, top, anywhere)
    values = torch.randn(nnz, generator=g).to(torch.bfloat16)
    csr = (indptr.cuda(), indices.cuda(), values.cuda())
    got = sparse_decode(*csr, W, b)
    assert torch.equal(got, sparse_decode(*csr, W, b, config={"BLOCK_NNZ": 64, "BLOCK_D": 1 << 20}))
    ip = indptr.numpy()
    for r in (0, 77, M - 1):
        cols = indices[ip[r]:ip[r + 1]].long()
        sub_w = W[cols.cuda()].cpu().double().numpy()  # only this row's decoder rows
        want = ocsr.sparse_decode(np.array([0, len(cols)]), np.arange(len(cols), dtype=np.int32),
                                  values[ip[r]:ip[r + 1]].double().numpy(), sub_w, b.cpu().double().numpy())
        torch.testing.assert_close(got[r:r + 1].cpu().double(), torch.from_numpy(want),
                                   atol=4 * TOL[torch.bfloat16], rtol=TOL[torch.bfloat16])


def test_csr_to_dense_round_trip_and_duplicates():
    f = torch.relu(torch.randn(37, 129) - 1.0).cuda()
    assert torch.equal(csr_to_dense(*dense_to_csr(f), 129), f)
    indptr = torch.tensor([0, 3], dtype=torch.int64, device="cuda")
    indices = torch.tensor([2, 5, 2], dtype=torch.int32, device="cuda")
    values = torch.tensor([1.0, 2.0, 0.5], device="cuda")
    dense = csr_to_dense(indptr, indices, values, 8).cpu()
    assert dense.tolist() == [[0, 0, 1.5, 0, 0, 2.0, 0, 0]]


# ----------------------------------------------------------------------------- top-k and ops


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("N,k", [(3000, 17), (3000, 1000), (3001, 1000), (30000, 33)])
def test_topk_rows_vector_and_uncached_rows(dtype, N, k):
    """Rows of 16-B chunks cached in LDS (N=3000), too long for the LDS copy (N=30000), or
    with a row stride that is not a multiple of 16 B (N=3001, the element-wise kernel); each
    also as a view one column narrower, which leaves a tail of fewer than 16 B on the
    chunked rows. Negative values, mostly-zero rows, all-zero rows and ties at the cut."""
    g = torch.Generator().manual_seed(N + k)
    f = torch.randn(6, N, generator=g)
    f[1] = torch.relu(f[1] - 2.5)  # mostly zeros: the cut falls inside the zeros
    f[2] = 0.0
    f[3, ::7] = 0.75  # many ties at one value
    f[4] = torch.round(f[4] * 2) / 2  # few distinct values
    f = f.to(dtype)
    fg = f.cuda()
    for src, ref in ((fg, f), (fg[:, :-1], f[:, :-1])):  # the GPU view keeps the row stride
        kk = min(k, src.shape[1])
        vals, idx = topk_rows(src, kk)
        want_v, want_i = ocsr.topk_rows(ref.double().numpy(), kk)
        np.testing.assert_array_equal(vals.cpu().double().numpy(), want_v)
        np.testing.assert_array_equal(idx.cpu().numpy(), want_i)


@pytest.mark.parametrize("dtype", DTYPES)
def test_topk_rows(dtype):
    f = torch.relu(torch.randn(50, 3000)).to(dtype)
    f[3] = 0  # all ties
    f[4, :10] = 1.0  # ties at the cut
    vals, idx = topk_rows(f.cuda(), 17)
    want_v, want_i = ocsr.topk_rows(f.double().numpy(), 17)
    np.testing.assert_array_equal(vals.cpu().double().numpy(), want_v)
    np.testing.assert_array_equal(idx.cpu().numpy(), want_i)  # ties by increasing column
    top = f.cuda().topk(17, dim=-1)
    assert torch.equal(vals, top.values)  # same values as torch.topk, sorted descending


def test_topk_golden():
    with np.load(GOLDEN / "topk.npz", allow_pickle=False) as z:
        g = {k: z[k] for k in z.files}
    vals, idx = topk_rows(torch.from_numpy(g["f"]).cuda(), int(g["k"]))
    np.testing.assert_array_equal(vals.cpu().double().numpy(), g["values"])
    np.testing.assert_array_equal(idx.cpu().numpy(), g["cols"])


@pytest.mark.parametrize("activation", ["relu", "jumprelu", "topk"])
def test_ops_match_reference(activation):
    # test_kernels.py:82-89 at 1e-4, plus the stricter fp32 bar
    p = make_params(40, 150, activation, torch.float32)
    x = torch.randn(33, 40)
    sae = Sae(gpu(p), activation, k=8)
    xg = x.cuda()
    want = oref.encode(x, p["W_enc"], p["b_enc"], p["b_dec"], p["threshold"], activation, 8)
    torch.testing.assert_close(saeflow_amd.encode(sae, xg).cpu(), want, atol=1e-4, rtol=1e-4)
    csr = saeflow_amd.encode_sparse(sae, xg)
    assert csr[0].dtype == torch.int64 and csr[1].dtype == torch.int32
    torch.testing.assert_close(csr_to_dense(*csr, 150).cpu(), want, atol=1e-4, rtol=1e-4)
    want_fwd = oref.forward(x, p["W_enc"], p["b_enc"], p["b_dec"], p["W_dec"], p["threshold"], activation, 8)
    torch.testing.assert_close(saeflow_amd.forward(sae, xg).cpu(), want_fwd, atol=1e-4, rtol=1e-4)


def test_sae_module_runs_on_gpu_kernels():
    torch.manual_seed(0)
    sae = saeflow_amd.SAE(64, 256, "jumprelu", device="cuda")
    sae.b_enc.normal_(0, 0.1)
    sae.b_dec.normal_(0, 0.1)
    sae.threshold.uniform_(0.0, 0.5)
    x = torch.randn(20, 64, device="cuda")
    p = {k: getattr(sae, k).detach().cpu() for k in ("W_enc", "b_enc", "b_dec", "W_dec", "threshold")}
    want = oref.forward(x.cpu(), p["W_enc"], p["b_enc"], p["b_dec"], p["W_dec"], p["threshold"], "jumprelu")
    torch.testing.assert_close(sae(x).cpu(), want, atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(sae.encode_pre(x).cpu(), oref.encode_pre(x.cpu(), p["W_enc"], p["b_enc"], p["b_dec"]),
                               atol=1e-4, rtol=1e-4)


# ----------------------------------------------------------------------------- benchmark-size properties


def _sample_rows_check(sae, x, got_f, rows, dtype):
    p = {k: getattr(sae, k).cpu() for k in ("W_enc", "b_enc", "b_dec")}
    thr = sae.threshold.cpu() if sae.threshold is not None else None
    pre = oref.encode_pre(x[rows].cpu(), p["W_enc"], p["b_enc"], p["b_dec"], dtype=torch.float32).double()
    want = oref.activate(pre, sae.activation, thr)
    cut = pre - (thr.double() if sae.activation == "jumprelu" else 0)
    tol = TOL[dtype] * (1 + pre.abs().max())
    keep = cut.abs() > tol
    torch.testing.assert_close(got_f[rows].cpu().double()[keep], want[keep], atol=float(tol), rtol=TOL[dtype])


@pytest.mark.parametrize("name,T,d_sae", [("C1", None, None), ("C2", 4096, None), ("C3", 4096, None),
                                         ("C5", 1024, 131072)])
def test_pipeline_properties_at_benchmark_shapes(name, T, d_sae):
    sae, x, meta = workloads.make(name, T=T, d_sae=d_sae, device="cuda")
    dtype = meta["dtype"]
    M, N = x.shape[0], sae.W_enc.shape[1]
    row_nnz = torch.zeros(M, device="cuda", dtype=torch.int32)
    f = fused_encode(x, sae.W_enc, sae.b_enc, sae.b_dec, sae.threshold, sae.activation, row_nnz=row_nnz)
    assert torch.equal(row_nnz, torch.count_nonzero(f, dim=1).int())
    l0 = row_nnz.float().mean().item()
    assert 0.5 * (meta["l0_expected"] or 60) < l0 < 2 * (meta["l0_expected"] or 70)
    rows = torch.arange(0, M, max(1, M // 48))
    _sample_rows_check(sae, x, f, rows, dtype)
    indptr, indices, values = dense_to_csr(f, row_nnz)
    # round trip dense -> CSR -> dense is exact
    assert torch.equal(csr_to_dense(indptr, indices, values, N), f)
    _check_decode_properties(indptr, indices, values, sae.W_dec)
    # canonical: indices strictly increasing inside every row
    same_row = torch.repeat_interleave(torch.arange(M, device="cuda"), torch.diff(indptr))
    inc = indices[1:] > indices[:-1]
    assert bool((inc | (same_row[1:] != same_row[:-1])).all())
    # decode on sampled rows against the fp64 oracle of the same CSR
    out = sparse_decode(indptr, indices, values, sae.W_dec, sae.b_dec)
    ip = indptr.cpu().numpy()
    sub = rows.numpy()
    sub_ip = np.concatenate([[0], np.cumsum(ip[sub + 1] - ip[sub])])
    sel = np.concatenate([np.arange(ip[r], ip[r + 1]) for r in sub])
    want = ocsr.sparse_decode(sub_ip, indices.cpu().numpy()[sel], values.cpu().double().numpy()[sel],
                              sae.W_dec.cpu().double().numpy(), sae.b_dec.cpu().double().numpy())
    tol = TOL[dtype]
    torch.testing.assert_close(out[rows].cpu().double(), torch.from_numpy(want), atol=4 * tol, rtol=tol)
    # determinism: a second run is bit-identical
    row_nnz2 = torch.zeros(M, device="cuda", dtype=torch.int32)
    f2 = fused_encode(x, sae.W_enc, sae.b_enc, sae.b_dec, sae.threshold, sae.activation, row_nnz=row_nnz2)
    assert torch.equal(f2, f) and torch.equal(row_nnz2, row_nnz)
    assert torch.equal(sparse_decode(indptr, indices, values, sae.W_dec, sae.b_dec), out)


@pytest.mark.parametrize("case", range(24))
def test_random_shapes_end_to_end(case):
    """Seeded random shapes (M up to 600, d_in up to 300, d_sae up to 1200: ragged tiles, odd
    widths, K below one K-step), each dtype and activation, through the whole path: encode
    against the oracle with its counts, dense -> CSR bit-exact against torch's to_sparse_csr,
    decode of that CSR against the fp64 oracle."""
    g = torch.Generator().manual_seed(1000 + case)

    def rnd(lo, hi):
        return int(torch.randint(lo, hi + 1, (1,), generator=g))

    M, K, N = rnd(1, 600), rnd(1, 300), rnd(1, 1200)
    dtype = DTYPES[case % 3]
    activation = ("relu", "jumprelu")[(case // 3) % 2]
    p = make_params(K, N, activation, dtype, seed=case)
    x = torch.randn(M, K, generator=g).to(dtype)
    q = gpu(p)
    row_nnz = torch.zeros(M, device="cuda", dtype=torch.int32)
    f = fused_encode(x.cuda(), q["W_enc"], q["b_enc"], q["b_dec"], q["threshold"], activation, row_nnz=row_nnz)
    check_encode(f, x, p, activation, dtype)
    assert torch.equal(row_nnz.cpu(), torch.count_nonzero(f, dim=1).int().cpu())
    indptr, indices, values = dense_to_csr(f, row_nnz)
    want = f.cpu().to_sparse_csr()
    bits = torch.int32 if dtype == torch.float32 else torch.int16
    assert torch.equal(indptr.cpu(), want.crow_indices())
    assert torch.equal(indices.long().cpu(), want.col_indices())
    assert torch.equal(values.cpu().view(bits), want.values().view(bits))
    out = sparse_decode(indptr, indices, values, q["W_dec"], q["b_dec"])
    ref = ocsr.sparse_decode(indptr.cpu().numpy(), indices.cpu().numpy(), values.cpu().double().numpy(),
                             p["W_dec"].double().numpy(), p["b_dec"].double().numpy())
    torch.testing.assert_close(out.cpu().double(), torch.from_numpy(ref), atol=8 * TOL[dtype], rtol=TOL[dtype])


def _check_decode_properties(indptr, indices, values, W_dec):
    """Two properties of the decode sums that hold exactly at any size, over every row:
    doubling the values doubles every fp32 output (scaling by 2 is exact in each product, each
    partial sum and the final rounding), and decoding the tokens in reverse order reverses the
    output rows (a token's pairs are summed in an order that depends only on that token's own
    entries, and padding pairs add exact zeros)."""
    M = indptr.numel() - 1
    out = sparse_decode(indptr, indices, values, W_dec, out_dtype=torch.float32)
    assert bool(torch.isfinite(out).all())
    assert torch.equal(sparse_decode(indptr, indices, values * 2, W_dec, out_dtype=torch.float32), out * 2)
    lens = torch.diff(indptr).long().flip(0)
    rev_ip = torch.zeros(M + 1, dtype=indptr.dtype, device=indptr.device)
    rev_ip[1:] = torch.cumsum(lens, 0)
    starts = indptr[:-1].long().flip(0)
    src = torch.repeat_interleave(starts - rev_ip[:-1].long(), lens) + torch.arange(int(lens.sum()),
                                                                                    device=indptr.device)
    out_rev = sparse_decode(rev_ip, indices[src], values[src], W_dec, out_dtype=torch.float32)
    assert torch.equal(out_rev, out.flip(0))


@pytest.mark.parametrize("name", ["C3", "C5"])
def test_pipeline_full_size(name):
    """The headline configuration C3 at its real size (T = 16384, d_sae = 65536, dense f
    2.15 GB) and C5 (d_sae = 2^20: W_enc and W_dec 4.8 GB each, dense f 8.6 GB, offsets past
    2^31 elements): counts equal the nonzeros, sampled rows against the CPU oracle, exact CSR
    round trip, every row through the roll and decode properties, and decode of sampled rows
    against the oracle."""
    sae, x, meta = workloads.make(name, device="cuda")
    M, N = x.shape[0], sae.W_enc.shape[1]
    if name == "C5":
        assert N == 1 << 20 and M * N >= 2 ** 32
    else:
        assert (M, N) == (16384, 65536)
    row_nnz = torch.zeros(M, device="cuda", dtype=torch.int32)
    f = fused_encode(x, sae.W_enc, sae.b_enc, sae.b_dec, sae.threshold, sae.activation, row_nnz=row_nnz)
    assert torch.equal(row_nnz, torch.count_nonzero(f, dim=1).int())
    l0 = row_nnz.float().mean().item()
    assert 0.5 * meta["l0_expected"] < l0 < 2 * meta["l0_expected"]
    rows = torch.tensor([0, 1, 1777, M // 2 + 3, M - 2, M - 1])
    _sample_rows_check(sae, x, f, rows, torch.bfloat16)
    indptr, indices, values = dense_to_csr(f, row_nnz)
    assert int(indptr[-1]) == int(row_nnz.sum())
    assert torch.equal(csr_to_dense(indptr, indices, values, N), f)
    # every row, through a property that holds at any size: rolling the tokens by one (so no
    # row keeps its place inside a 256-row tile) rolls f and the counts bit for bit, since each
    # output element sums the same products in the same K order wherever its row sits
    row_nnz_r = torch.zeros(M, device="cuda", dtype=torch.int32)
    f_r = fused_encode(torch.roll(x, 1, 0), sae.W_enc, sae.b_enc, sae.b_dec, sae.threshold, sae.activation,
                       row_nnz=row_nnz_r)
    assert torch.equal(f_r, torch.roll(f, 1, 0)) and torch.equal(row_nnz_r, torch.roll(row_nnz, 1, 0))
    del f, f_r
    _check_decode_properties(indptr, indices, values, sae.W_dec)
    out = sparse_decode(indptr, indices, values, sae.W_dec, sae.b_dec)
    ip = indptr.cpu().numpy()
    for r in rows.tolist():
        cols = indices[ip[r]:ip[r + 1]].long()
        sub_w = sae.W_dec[cols].cpu().double().numpy()  # only this row's decoder rows
        want = ocsr.sparse_decode(np.array([0, len(cols)]), np.arange(len(cols), dtype=np.int32),
                                  values[ip[r]:ip[r + 1]].cpu().double().numpy(), sub_w,
                                  sae.b_dec.cpu().double().numpy())
        torch.testing.assert_close(out[r:r + 1].cpu().double(), torch.from_numpy(want),
                                   atol=4 * TOL[torch.bfloat16], rtol=TOL[torch.bfloat16])


def test_topk_pipeline_at_c4_width():
    sae, x, meta = workloads.make("C4", T=512, device="cuda")
    csr = saeflow_amd.encode_sparse(sae, x)
    k = sae.k
    assert csr[0].tolist() == list(range(0, 512 * k + 1, k))
    f = fused_encode(x, sae.W_enc, sae.b_enc, sae.b_dec, activation="relu")
    top = f.topk(k, dim=-1)
    vals = csr[2].view(512, k)
    assert torch.equal(vals, top.values)
    # the selected columns hold exactly the selected values
    assert torch.equal(f.gather(1, csr[1].view(512, k).long()), vals)
    out = saeflow_amd.forward(sae, x)
    dense = torch.zeros_like(f).scatter_(1, csr[1].view(512, k).long(), vals)
    want = dense[:64].double().cpu() @ sae.W_dec.double().cpu() + sae.b_dec.double().cpu()
    torch.testing.assert_close(out[:64].cpu().double(), want, atol=2e-2, rtol=5e-3)


# ----------------------------------------------------------------------------- TopK against the oracle


def _oracle_pre_rows(sae, x, rows, chunk=16384):
    """float64 pre-activation of the sampled rows from the same rounded inputs (reference.py:36-37),
    in column chunks so the float64 copy of W_enc stays small."""
    xs = x[rows].cpu()
    N = sae.W_enc.shape[1]
    out = torch.empty(len(rows), N, dtype=torch.float64)
    for c0 in range(0, N, chunk):
        sl = slice(c0, min(N, c0 + chunk))
        out[:, sl] = oref.encode_pre(xs, sae.W_enc[:, sl].cpu(), sae.b_enc[sl].cpu(), sae.b_dec.cpu(),
                                     dtype=torch.float64)
    return out


def _check_topk_rows_against_oracle(sae, x, values, indices, rows, dtype):
    """TopK selections of sampled rows against the CPU oracle: relu of the float64
    pre-activation, then the row top-k with this build's tie rule (oracle.csr.topk_rows:
    values descending, equal values by increasing column).

    The GPU rounds fp32 sums to the value dtype, so selections may differ from the oracle's
    only among features within atol of the oracle's k-th value (the near-cut exclusion of
    test_kernels.py:39-43, applied at the top-k cut). Checked:
      - each selected value is within atol + rtol*|want| of relu(pre) at its column;
      - every feature above kth + atol is selected, none below kth - atol is;
      - the GPU order is values descending, equal values by increasing column (exact).
    The reference's oracle takes top-k of pre and then relu (reference.py:45-46) where ops
    relus first (ops.py:15-16); the two agree whenever a row has at least k positive
    pre-activations, which is asserted for every sampled row (b_enc = -2.8 leaves about
    d_sae * 0.0026 positives per row)."""
    k = values.shape[1]
    pre = _oracle_pre_rows(sae, x, rows)
    want = torch.relu(pre)
    assert bool(((pre > 0).sum(1) >= k).all()), "a sampled row has fewer than k positives"
    rtol = TOL[dtype]
    atol = rtol * (1 + pre.abs().max().item())
    got_v = values[rows].cpu().double()
    got_i = indices[rows].cpu().long()
    at_cols = want.gather(1, got_i)
    assert bool(((got_v - at_cols).abs() <= atol + rtol * at_cols.abs()).all())
    want_v, want_i = ocsr.topk_rows(want.numpy(), k)
    kth = torch.from_numpy(want_v[:, k - 1])
    for r in range(len(rows)):
        sel = set(got_i[r].tolist())
        must = torch.nonzero(want[r] > kth[r] + atol).flatten().tolist()
        assert set(must) <= sel, f"row {int(rows[r])}: a feature clearly above the k-th value was not selected"
        assert bool((want[r, got_i[r]] >= kth[r] - atol).all()), f"row {int(rows[r])}: a feature below the cut"
        # where no feature sits near the cut the selection is the oracle's exactly
        if int(((want[r] - kth[r]).abs() <= atol).sum()) == 1:
            assert sel == set(want_i[r].tolist())
    # order: descending values, ties by increasing column
    gv, gi = values.cpu().double(), indices.cpu().long()
    assert bool((gv[:, 1:] <= gv[:, :-1]).all())
    tie = gv[:, 1:] == gv[:, :-1]
    assert bool((~tie | (gi[:, 1:] > gi[:, :-1])).all())


def test_topk_c4_full_size_against_oracle():
    """C4 at its real size (fp16, d_in 4096, d_sae 131072, T 8192, k 32) through
    encode_sparse, which takes the floor-filtered row-candidate select at this width:
    sampled rows against the CPU oracle, and over every row the size-independent
    properties of a top-k of the dense HIP encode (selected columns hold exactly the dense
    values, nothing unselected above the k-th value)."""
    sae, x, meta = workloads.make("C4", device="cuda")
    M, N, k = x.shape[0], sae.W_enc.shape[1], sae.k
    assert (M, N, k) == (8192, 131072, 32)
    indptr, indices, values = saeflow_amd.encode_sparse(sae, x)
    assert torch.equal(indptr, torch.arange(0, M * k + 1, k, device="cuda", dtype=torch.int64))
    values, indices = values.view(M, k), indices.view(M, k)
    rows = torch.tensor([0, 1, 2, 777, 4095, 4096, 6001, 8190, 8191])
    _check_topk_rows_against_oracle(sae, x, values, indices, rows, torch.float16)
    f = fused_encode(x, sae.W_enc, sae.b_enc, sae.b_dec, activation="relu")
    assert torch.equal(f.gather(1, indices.long()), values)
    kth = values[:, k - 1:k]
    assert bool(((f > kth).sum(1) < k).all()) and bool(((f >= kth).sum(1) >= k).all())


def test_topk_forced_row_path_against_oracle():
    """The row-candidate TopK (floor from the first S features, filtered lists, list select)
    at a quarter of C4's width, against the oracle; also with a capacity about half of the
    rows overflow, so those rows go through the per-row dense fallback."""
    from saeflow_amd import ops
    sae, x, meta = workloads.make("C4", T=1024, d_sae=32768, device="cuda")
    assert ops.ROW_PATHS and sae.W_enc.shape[1] >= ops.TOPK_MIN_FEATURES
    rows = torch.tensor([0, 5, 511, 1023])
    v, i = ops._topk_rows(sae, x)
    _check_topk_rows_against_oracle(sae, x, v, i, rows, torch.float16)
    saved = ops.TOPK_CAP
    try:
        ops.TOPK_CAP = 256  # lists hold about k * N / S = 256 entries: about half overflow
        v2, i2 = ops._topk_rows(sae, x)
    finally:
        ops.TOPK_CAP = saved
    assert torch.equal(i2, i) and torch.equal(v2, v)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("N,k", [(3000, 1025), (5000, 2048), (3001, 3001), (20000, 4100)])
def test_topk_rows_above_the_lds_limit(dtype, N, k):
    """k above 1024 (the LDS-sorted limit): selection staged and sorted in the output rows;
    same ties, order and values as the oracle's top-k (f.topk has no bound on k, ops.py:16)."""
    g = torch.Generator().manual_seed(N + k)
    f = torch.randn(5, N, generator=g)
    f[1] = torch.relu(f[1] - 1.5)  # the cut inside the zeros
    f[2, ::3] = 0.5  # many ties
    f[3] = torch.round(f[3] * 4) / 4
    f = f.to(dtype)
    for src in (f.cuda(), f.cuda()[:, ::1][:, : N - 1]):
        ref = src.cpu()
        kk = min(k, src.shape[1])
        vals, idx = topk_rows(src, kk)
        want_v, want_i = ocsr.topk_rows(ref.double().numpy(), kk)
        np.testing.assert_array_equal(idx.cpu().numpy(), want_i)
        np.testing.assert_array_equal(vals.cpu().double().numpy(), want_v)


def test_csr_to_dense_long_rows():
    """Rows of 65536 entries: canonical (strictly increasing), permuted (distinct columns in
    any order), and repeating columns (summed in entry order), against the oracle."""
    N = 1 << 17
    g = torch.Generator().manual_seed(5)
    cols0 = torch.randperm(N, generator=g)[:65536].sort().values
    cols1 = torch.randperm(N, generator=g)[:65536]
    cols2 = torch.randint(0, 4096, (65536,), generator=g)
    indices = torch.cat([cols0, cols1, cols2]).int()
    values = torch.randint(-8, 8, (3 * 65536,), generator=g).float() / 8  # sums exact in fp32
    indptr = torch.tensor([0, 65536, 131072, 196608], dtype=torch.int64)
    got = csr_to_dense(indptr.cuda(), indices.cuda(), values.cuda(), N).cpu()
    want = ocsr.csr_to_dense(indptr.numpy(), indices.numpy(), values.numpy(), N)
    np.testing.assert_array_equal(got.double().numpy(), want)


def test_fixed_width_to_dense_is_scatter():
    """The TopK scatter zeros.scatter_(-1, indices, values) (ops.py:21-25) for rows of k = 2000
    distinct columns in value order (no longer the serial path) and for k = 7: every value's
    bits land as they are, -0.0 included, bit-equal to torch's scatter_."""
    from saeflow_amd.kernels import fixed_width_to_dense
    g = torch.Generator().manual_seed(9)
    N = 8192
    for k in (7, 2000):
        idx = torch.stack([torch.randperm(N, generator=g)[:k] for _ in range(5)]).int()
        vals = torch.randn(5, k, generator=g).to(torch.bfloat16)
        vals[0, :3] = -0.0
        vals[3, 5 % k] = -0.0
        want = torch.zeros(5, N, dtype=torch.bfloat16).scatter_(-1, idx.long(), vals)
        got = fixed_width_to_dense(idx.cuda(), vals.cuda(), N).cpu()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), k


@pytest.mark.parametrize("cfg", [{"BLOCK_NNZ": 16, "BLOCK_D": 128}, {"BLOCK_NNZ": 32, "BLOCK_D": 512},
                                 {"BLOCK_NNZ": 64, "BLOCK_D": 1024}, {"BLOCK_NNZ": 8, "BLOCK_D": 100000}])
@pytest.mark.parametrize("dtype", DTYPES)
def test_sparse_decode_config_changes_speed_only(cfg, dtype):
    """sparse_decode(config=...) (decode.py:101) runs the one-row-per-wavefront kernel with that
    slab width (the default at d_in = 2304 is the line-slab kernel); every output sums its
    entries in entry order, so the result is bit-identical to the default."""
    p = make_params(2304, 1024, "relu", dtype)
    f = torch.relu(torch.randn(40, 1024) - 1.5).to(dtype)
    indptr, indices, values = dense_to_csr(f.cuda())
    W, b = p["W_dec"].cuda(), p["b_dec"].cuda()
    want = sparse_decode(indptr, indices, values, W, b)
    got = sparse_decode(indptr, indices, values, W, b, config=cfg)
    assert torch.equal(got, want)
    ref = ocsr.sparse_decode(indptr.cpu().numpy(), indices.cpu().numpy(), values.cpu().double().numpy(),
                             p["W_dec"].double().numpy(), p["b_dec"].double().numpy())
    torch.testing.assert_close(got.cpu().double(), torch.from_numpy(ref), atol=4 * TOL[dtype], rtol=TOL[dtype])
    with pytest.raises(ValueError, match="BLOCK_NNZ"):
        sparse_decode(indptr, indices, values, W, b, config={"BLOCK_D": 128})


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("N,k", [(40, 12), (4000, 300), (3001, 2000)])
def test_topk_rows_zero_signs_and_nans(dtype, N, k):
    """-0.0 ties with +0.0 and NaN of either sign ranks first, as f.topk compares them
    (oracle.csr.topk_rows states the rule); the written values are the input's own bits."""
    g = torch.Generator().manual_seed(N)
    f = torch.round(torch.randn(4, N, generator=g) * 2) / 2  # many +-0.0 and ties
    f[1, ::5] = float("nan")
    f[1, 3::7] = -float("nan")
    f[2] = -0.0
    f[2, ::3] = 0.0
    f = f.to(dtype)
    for src in (f.cuda(), f.cuda()[:, ::2]):  # contiguous rows and a strided view
        ref = src.cpu()
        kk = min(k, src.shape[1])
        vals, idx = topk_rows(src, kk)
        want_v, want_i = ocsr.topk_rows(ref.double().numpy(), kk)
        np.testing.assert_array_equal(idx.cpu().numpy(), want_i)
        got_bits = ocsr.to_bits(vals)
        want_bits = ocsr.to_bits(ref.gather(1, idx.cpu().long()))
        np.testing.assert_array_equal(got_bits, want_bits)
