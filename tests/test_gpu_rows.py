"""GPU: the row-candidate encode (no dense output) against the dense path and the oracle.

The row-candidate path must reproduce the dense path bit for bit: the candidates of a row
are exactly the nonzeros fused_encode stores (same columns, same rounded values), their
count is the row_nnz count, rows_to_csr equals dense_to_csr of the dense features, and the
TopK select over floor-filtered candidates equals the dense top-k (values, columns and tie
order). Rows whose candidate list overflows are encoded again alone through the dense path,
with identical results.
"""

import numpy as np
import pytest
import torch

import saeflow_amd
from oracle import csr as ocsr
from saeflow_amd import ops, workloads
from saeflow_amd.kernels import (dense_to_csr, encode_gather, encode_rows, exclusive_scan, fused_encode,
                                 overflow_rows, rows_to_csr, rows_topk, topk_gather, topk_rows)

pytestmark = pytest.mark.gpu

SHAPES = [(1, 16, 32), (37, 50, 129), (300, 128, 520), (257, 64, 264), (16, 2304, 512), (700, 96, 3000)]
DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def params(d_in, d_sae, activation, dtype, seed=0, b_shift=0.0):
    g = torch.Generator().manual_seed(seed)
    W_dec = torch.randn(d_sae, d_in, generator=g)
    W_dec /= W_dec.norm(dim=1, keepdim=True)
    p = dict(W_enc=W_dec.T.contiguous() * 3.0, b_enc=torch.randn(d_sae, generator=g) * 0.1 + b_shift,
             b_dec=torch.randn(d_in, generator=g) * 0.1,
             threshold=torch.rand(d_sae, generator=g) * 0.5 if activation == "jumprelu" else None)
    return {k: (v.to(dtype).cuda() if v is not None else None) for k, v in p.items()}


def candidates_as_sets(cnt, idx, val):
    out = []
    c = cnt.cpu().numpy()
    ii = idx.cpu().numpy()
    vv = ocsr.to_bits(val)
    for m in range(len(c)):
        n = min(int(c[m]), ii.shape[1])
        out.append(sorted(zip(ii[m, :n].tolist(), vv[m, :n].tolist())))
    return out


@pytest.mark.parametrize("activation", ["relu", "jumprelu"])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", SHAPES)
def test_candidates_are_the_stored_nonzeros(shape, dtype, activation):
    M, d_in, d_sae = shape
    p = params(d_in, d_sae, activation, dtype, b_shift=-0.5)
    x = torch.randn(M, d_in).to(dtype).cuda()
    row_nnz = torch.zeros(M, device="cuda", dtype=torch.int32)
    f = fused_encode(x, p["W_enc"], p["b_enc"], p["b_dec"], p["threshold"], activation, row_nnz=row_nnz)
    cap = d_sae  # never overflows
    cnt, idx, val = encode_rows(x, p["W_enc"], p["b_enc"], p["b_dec"], p["threshold"], activation, cap=min(cap, 4096))
    assert torch.equal(cnt, row_nnz)
    fb = ocsr.to_bits(f)
    nzm = (f != 0).cpu().numpy()
    want = [sorted((int(c), int(fb[m, c])) for c in np.flatnonzero(nzm[m])) for m in range(M)]
    assert candidates_as_sets(cnt, idx, val) == want
    # CSR through the candidates equals the dense compaction exactly
    indptr = exclusive_scan(cnt)
    nnz = int(indptr[-1])
    indices, values = rows_to_csr(cnt, idx, val, indptr, nnz)
    ip2, ind2, val2 = dense_to_csr(f, row_nnz)
    assert torch.equal(indptr, ip2) and torch.equal(indices, ind2)
    assert np.array_equal(ocsr.to_bits(values), ocsr.to_bits(val2))


@pytest.mark.parametrize("floor", [False, True])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(256, 64, 256), (512, 96, 768), (1536, 192, 2304), (4096, 320, 8448)])
def test_persistent_row_candidates_equal_one_tile_per_workgroup(shape, dtype, floor):
    """Whole-tile shapes run the row-candidate epilogues in the persistent 8-wave kernel; one
    more token row runs them one workgroup per tile. The first M rows' candidate sets (columns
    and value bits) and counts agree, with and without a row floor (relu), and the counts equal
    the dense encode's row counts. One tile and 2 x 3 tiles leave XCDs with no tile."""
    M, d_in, d_sae = shape
    for activation in ("relu",) if floor else ("relu", "jumprelu"):  # a row floor goes with relu
        p = params(d_in, d_sae, activation, dtype, b_shift=-0.5)
        x = torch.randn(M + 1, d_in).to(dtype).cuda()
        rf = torch.randn(M + 1, device="cuda") * 0.5 + 0.5 if floor else None
        got = encode_rows(x[:M], p["W_enc"], p["b_enc"], p["b_dec"], p["threshold"], activation, cap=4096,
                          row_floor=rf[:M] if floor else None)
        ref = encode_rows(x, p["W_enc"], p["b_enc"], p["b_dec"], p["threshold"], activation, cap=4096,
                          row_floor=rf)
        assert torch.equal(got[0], ref[0][:M]), activation
        assert candidates_as_sets(*got) == candidates_as_sets(ref[0][:M], ref[1][:M], ref[2][:M]), activation
        if not floor:
            row_nnz = torch.zeros(M, device="cuda", dtype=torch.int32)
            f = fused_encode(x[:M], p["W_enc"], p["b_enc"], p["b_dec"], p["threshold"], activation, row_nnz=row_nnz)
            assert torch.equal(got[0], row_nnz)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rows_to_csr_sorts_every_list_length(dtype):
    """Lists of up to 256 candidates are sorted by one wavefront in registers, longer ones by a
    block in LDS: lengths around both limits (0, 1, 63-65, 255-257, 700, the capacity 1024) and
    an overflowed row (count above the capacity: its segment is left alone) give each row its
    columns in increasing order with the matching values."""
    g = torch.Generator().manual_seed(7)
    cap, N = 1024, 5000
    lens = [0, 1, 63, 64, 65, 255, 256, 257, 700, 1024, 1500, 40, 3, 130]
    M = len(lens)
    cnt = torch.tensor(lens, dtype=torch.int32)
    idx = torch.full((M, cap), -7, dtype=torch.int32)
    val = torch.zeros(M, cap, dtype=dtype)
    want_idx, want_val = [], []
    for m, n in enumerate(lens):
        if n > cap:
            continue
        cols = torch.randperm(N, generator=g)[:n].to(torch.int32)
        vals = torch.randn(n, generator=g).to(dtype)
        idx[m, :n], val[m, :n] = cols, vals
        order = torch.argsort(cols.long())
        want_idx.append(cols[order])
        want_val.append(vals[order])
    seg = torch.tensor([0 if n > cap else n for n in lens])
    indptr = torch.zeros(M + 1, dtype=torch.int64)
    indptr[1:] = torch.cumsum(seg, 0)
    nnz = int(indptr[-1])
    got_i, got_v = rows_to_csr(cnt.cuda(), idx.cuda(), val.cuda(), indptr.cuda(), nnz)
    assert torch.equal(got_i.cpu(), torch.cat(want_idx))
    assert torch.equal(got_v.cpu().view(torch.int16 if dtype == torch.bfloat16 else torch.int32),
                       torch.cat(want_val).view(torch.int16 if dtype == torch.bfloat16 else torch.int32))


def test_candidate_overflow_is_counted_and_capped():
    p = params(64, 1024, "relu", torch.bfloat16, b_shift=1.0)  # about 85% of the features fire
    x = torch.randn(40, 64).to(torch.bfloat16).cuda()
    row_nnz = torch.zeros(40, device="cuda", dtype=torch.int32)
    fused_encode(x, p["W_enc"], p["b_enc"], p["b_dec"], activation="relu", row_nnz=row_nnz)
    cnt, idx, val = encode_rows(x, p["W_enc"], p["b_enc"], p["b_dec"], activation="relu", cap=16)
    assert torch.equal(cnt, row_nnz) and int(cnt.min()) > 16
    # every written slot holds a real nonzero of its row (no slot past cap was touched)
    assert bool((idx >= 0).all()) and bool((idx < 1024).all())


def test_row_floor_keeps_values_at_or_above_it():
    p = params(96, 2048, "relu", torch.float16, b_shift=-0.2)
    x = torch.randn(64, 96).to(torch.float16).cuda()
    f = fused_encode(x, p["W_enc"], p["b_enc"], p["b_dec"], activation="relu")
    floor = torch.rand(64, device="cuda") * 0.8
    floor[3] = 0.0
    floor[5] = float(f[5].max())  # exactly the row maximum: keeps the maxima only
    cnt, idx, val = encode_rows(x, p["W_enc"], p["b_enc"], p["b_dec"], activation="relu", cap=2048, row_floor=floor)
    keep = (f > 0) & (f.float() >= floor[:, None])
    assert torch.equal(cnt, keep.sum(1).int())
    got = candidates_as_sets(cnt, idx, val)
    fb = ocsr.to_bits(f)
    for m in (0, 3, 5, 63):
        cols = np.flatnonzero(keep[m].cpu().numpy())
        assert got[m] == sorted((int(c), int(fb[m, c])) for c in cols)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_rows_topk_equals_dense_topk_with_floor_from_a_subset(dtype):
    M, d_in, N, k = 96, 128, 8192, 24
    p = params(d_in, N, "relu", dtype, b_shift=-0.8)
    x = torch.randn(M, d_in).to(dtype).cuda()
    f = fused_encode(x, p["W_enc"], p["b_enc"], p["b_dec"], activation="relu")
    want_v, want_i = topk_rows(f, k)
    S = 1024
    sub = fused_encode(x, p["W_enc"][:, :S], p["b_enc"][:S], p["b_dec"], activation="relu")
    floor = topk_rows(sub, k)[0][:, k - 1].float()
    cnt, idx, val = encode_rows(x, p["W_enc"], p["b_enc"], p["b_dec"], activation="relu", cap=4096, row_floor=floor)
    assert int(cnt.max()) <= 4096
    got_v, got_i = rows_topk(cnt, idx, val, k, N)
    assert torch.equal(got_i, want_i)
    assert np.array_equal(ocsr.to_bits(got_v), ocsr.to_bits(want_v))


def test_rows_topk_pads_rows_with_few_nonzeros():
    # rows with fewer than k positive values: zeros at the lowest free columns, as topk_rows
    M, d_in, N, k = 20, 32, 512, 40
    p = params(d_in, N, "relu", torch.bfloat16, b_shift=-6.0)
    x = torch.randn(M, d_in).to(torch.bfloat16).cuda()
    f = fused_encode(x, p["W_enc"], p["b_enc"], p["b_dec"], activation="relu")
    assert int((f > 0).sum(1).min()) < k
    want_v, want_i = topk_rows(f, k)
    cnt, idx, val = encode_rows(x, p["W_enc"], p["b_enc"], p["b_dec"], activation="relu", cap=512)
    got_v, got_i = rows_topk(cnt, idx, val, k, N)
    assert torch.equal(got_i, want_i)
    assert torch.equal(got_v, want_v)


def _with_paths(flag, cap=None, topk_cap=None):
    class Ctx:
        def __enter__(self):
            self.saved = (ops.ROW_PATHS, ops.ROW_CAP, ops.TOPK_CAP)
            ops.ROW_PATHS = flag
            if cap is not None:
                ops.ROW_CAP = cap
            if topk_cap is not None:
                ops.TOPK_CAP = topk_cap

        def __exit__(self, *exc):
            ops.ROW_PATHS, ops.ROW_CAP, ops.TOPK_CAP = self.saved
    return Ctx()


@pytest.mark.parametrize("name,T,d_sae", [("C2", 2048, None), ("C3", 1024, None), ("C1", None, None)])
def test_encode_sparse_row_path_equals_dense_path(name, T, d_sae):
    sae, x, meta = workloads.make(name, T=T, d_sae=d_sae, device="cuda")
    with _with_paths(False):
        want = saeflow_amd.encode_sparse(sae, x)
    with _with_paths(True):
        got = saeflow_amd.encode_sparse(sae, x)
    with _with_paths(True, cap=8):  # every list overflows: every row re-encoded densely, same result
        fell_back = saeflow_amd.encode_sparse(sae, x)
    for g in (got, fell_back):
        assert torch.equal(g[0], want[0]) and torch.equal(g[1], want[1])
        assert np.array_equal(ocsr.to_bits(g[2]), ocsr.to_bits(want[2]))


def test_topk_row_path_equals_dense_path_at_c4_width():
    sae, x, meta = workloads.make("C4", T=256, device="cuda")
    with _with_paths(False):
        want_v, want_i = ops._topk(sae, x)
    top = ops._topk_rows(sae, x)
    assert torch.equal(top[1], want_i) and torch.equal(top[0], want_v)
    with _with_paths(True, topk_cap=4):  # every list overflows: every row through the dense select
        fv, fi = ops._topk_rows(sae, x)
    assert torch.equal(fi, want_i) and torch.equal(fv, want_v)


def test_long_rows_are_reencoded_alone_at_c3_size(monkeypatch):
    """The headline workload (C3, T = 16384) with two planted long rows: one with x' scaled
    by 10 (about a third of its 65536 features fire) and one with a NaN input (every feature
    kept). Their lists overflow ROW_CAP; only those two rows are encoded again (one dense
    encode of 2 rows, no second encode of the batch), and the CSR equals the dense path's
    bit for bit."""
    sae, x, meta = workloads.make("C3", device="cuda")
    x = x.clone()
    x[777] = (sae.b_dec.float() + 10 * (x[777].float() - sae.b_dec.float())).to(x.dtype)
    x[9000, 5] = float("nan")
    with _with_paths(False):
        want = saeflow_amd.encode_sparse(sae, x)
    lens = torch.diff(want[0])
    assert int(lens[777]) > ops.ROW_CAP and int(lens[9000]) == 65536
    assert int((lens > ops.ROW_CAP).sum()) == 2
    calls = []
    real = ops.fused_encode

    def spy(xx, *a, **kw):
        calls.append(xx.shape[0])
        return real(xx, *a, **kw)

    monkeypatch.setattr(ops, "fused_encode", spy)
    got = saeflow_amd.encode_sparse(sae, x)
    assert calls == [2]
    assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])
    assert np.array_equal(ocsr.to_bits(got[2]), ocsr.to_bits(want[2]))


@pytest.mark.parametrize("narrow", [False, True])
def test_nan_input_rows_count_only_real_columns(narrow):
    # a NaN input makes its row all NaN (relu(NaN) = NaN, counted as nonzero by the
    # reference's f != 0); a ragged d_sae leaves padding columns in the last tile that must
    # not be counted
    M, d_in, N = 40, 64, 300
    p = params(d_in, N, "jumprelu", torch.bfloat16)
    x = torch.randn(M, d_in).to(torch.bfloat16)
    x[7, 3] = float("nan")
    x = x.cuda()
    cfg = {"BLOCK_M": 256, "BLOCK_N": 128, "BLOCK_K": 32, "GROUP_M": 2} if narrow else None
    row_nnz = torch.zeros(M, device="cuda", dtype=torch.int32)
    f = fused_encode(x, p["W_enc"], p["b_enc"], p["b_dec"], p["threshold"], "jumprelu", row_nnz=row_nnz, config=cfg)
    assert bool(torch.isnan(f[7]).all())
    assert torch.equal(row_nnz, torch.count_nonzero(f, dim=1).int())
    assert int(row_nnz[7]) == N
    cnt, idx, val = encode_rows(x, p["W_enc"], p["b_enc"], p["b_dec"], p["threshold"], "jumprelu", cap=512)
    assert torch.equal(cnt, row_nnz)
    assert sorted(idx[7, :N].tolist()) == list(range(N))


def _bits_equal(a, b):
    return np.array_equal(ocsr.to_bits(a), ocsr.to_bits(b))


def test_overflow_rows_lists_the_overflowed_rows_in_order():
    g = torch.Generator().manual_seed(3)
    for M in (1, 700, 1024, 1025, 5000):
        cnt = torch.randint(0, 40, (M,), generator=g, dtype=torch.int32)
        rows, n = overflow_rows(cnt.cuda(), 30)
        want = torch.nonzero(cnt > 30).flatten().to(torch.int32)
        assert int(n) == want.numel()
        assert torch.equal(rows[:want.numel()].cpu(), want)
    rows, n = overflow_rows(torch.zeros(0, dtype=torch.int32, device="cuda"), 4)
    assert int(n) == 0


@pytest.mark.parametrize("dtype", DTYPES)
def test_encode_gather_equals_the_dense_encode_of_the_rows(dtype):
    M, d_in, N = 600, 96, 1000
    p = params(d_in, N, "jumprelu", dtype, b_shift=-0.3)
    x = torch.randn(M, d_in).to(dtype).cuda()
    want = fused_encode(x, p["W_enc"], p["b_enc"], p["b_dec"], p["threshold"], "jumprelu")
    rows = torch.tensor([599, 3, 0, 257, 256, 77, 511, 2, 9, 300] * 30, dtype=torch.int32, device="cuda")
    for live, off, R in ((300, 0, 300), (300, 0, 512), (300, 100, 64), (0, 0, 256), (5, 0, 256), (300, 290, 32)):
        n = torch.tensor([live], dtype=torch.int32, device="cuda")
        got = encode_gather(x, p["W_enc"], p["b_enc"], p["b_dec"], rows, n, p["threshold"], "jumprelu",
                            row_off=off, out_rows=R)
        k = max(0, min(R, live - off))
        sel = rows[off:off + k].long()
        assert _bits_equal(got[:k], want[sel]), (live, off, R)


def test_encode_gather_rows_outside_x_encode_a_zero_row():
    # A row id outside [0, Mx) encodes a zero x' row, which is what a token equal to b_dec gives:
    # x' = cast(fp32(b_dec) - fp32(b_dec)) = 0.
    M, d_in, N = 40, 64, 700
    p = params(d_in, N, "jumprelu", torch.bfloat16, b_shift=0.4)
    x = torch.randn(M, d_in).to(torch.bfloat16).cuda()
    rows = torch.tensor([3, -1, M, 7, 1 << 30, -(1 << 30), 0], dtype=torch.int32, device="cuda")
    n = torch.tensor([rows.numel()], dtype=torch.int32, device="cuda")
    got = encode_gather(x, p["W_enc"], p["b_enc"], p["b_dec"], rows, n, p["threshold"], "jumprelu", out_rows=256)
    probe = torch.stack([x[3], p["b_dec"], p["b_dec"], x[7], p["b_dec"], p["b_dec"], x[0]])
    want = fused_encode(probe, p["W_enc"], p["b_enc"], p["b_dec"], p["threshold"], "jumprelu")
    assert bool((want[1] != 0).any())  # b_enc shifted up: the zero row has features
    assert _bits_equal(got[:rows.numel()], want)


def test_encode_gather_with_a_column_major_w_and_fp32_output():
    M, d_in, N = 300, 64, 520
    p = params(d_in, N, "relu", torch.bfloat16)
    Wk = p["W_enc"].T.contiguous().T  # d_in-contiguous: the K-major DMA path
    x = torch.randn(M, d_in).to(torch.bfloat16).cuda()
    want = fused_encode(x, Wk, p["b_enc"], p["b_dec"], out_dtype=torch.float32)
    rows = torch.arange(M - 1, -1, -1, dtype=torch.int32, device="cuda")
    n = torch.tensor([M], dtype=torch.int32, device="cuda")
    got = encode_gather(x, Wk, p["b_enc"], p["b_dec"], rows, n, row_off=0, out_rows=M, out_dtype=torch.float32)
    assert _bits_equal(got, want.flip(0))


def test_topk_gather_writes_only_the_mapped_rows():
    M, N, k = 50, 3000, 17
    f = torch.randn(M, N).to(torch.float16).cuda()
    want_v, want_i = topk_rows(f, k)
    M_out = 80
    fixed = [70, 5, 33, 0, 79, 12, 500, -1]  # 500 and -1 lie outside the output
    rest = [v for v in range(M_out) if v not in fixed][:M - len(fixed)]
    rows = torch.tensor(fixed + rest, dtype=torch.int32, device="cuda")  # distinct targets
    for live in (0, 3, 8, 50):
        vals = torch.full((M_out, k), 7.0, dtype=torch.float16, device="cuda")
        idx = torch.full((M_out, k), -5, dtype=torch.int32, device="cuda")
        n = torch.tensor([live], dtype=torch.int32, device="cuda")
        topk_gather(f, k, n, rows, vals, idx)
        touched = set()
        for i in range(live):
            o = int(rows[i])
            if 0 <= o < M_out:  # 500 and -1 are skipped
                touched.add(o)
                assert torch.equal(idx[o], want_i[i]) and _bits_equal(vals[o], want_v[i])
        for o in set(range(M_out)) - touched:
            assert bool((idx[o] == -5).all()) and bool((vals[o] == 7.0).all())


@pytest.mark.parametrize("dtype,k", [(torch.float32, 1500), (torch.bfloat16, 1025), (torch.float16, 300)])
def test_topk_gather_large_k_and_strided_rows(dtype, k):
    """The gathered top-k through each select kernel: k above 1024 (the selection sorted in the
    output row itself, here the mapped row) and a row-strided f view (element-wise kernel)."""
    M, N = 12, 4000
    base = torch.randn(M, N + 1).to(dtype).cuda()  # a row pitch of N + 1: rows not 16-B aligned
    f = base[:, :N] if k == 300 else base[:, :N].contiguous()
    want_v, want_i = topk_rows(f, k)
    rows = torch.tensor([3, 0, 7, 11, 2, 9], dtype=torch.int32, device="cuda")
    vals = torch.zeros(12, k, dtype=dtype, device="cuda")
    idx = torch.full((12, k), -1, dtype=torch.int32, device="cuda")
    n = torch.tensor([6], dtype=torch.int32, device="cuda")
    topk_gather(f, k, n, rows, vals, idx)
    for i, o in enumerate(rows.tolist()):
        assert torch.equal(idx[o], want_i[i]) and _bits_equal(vals[o], want_v[i]), (i, o)
    untouched = sorted(set(range(12)) - set(rows.tolist()))
    assert bool((idx[untouched] == -1).all())


def test_topk_row_path_redoes_overflowed_rows_in_chunks(monkeypatch):
    """Lists that overflow are redone densely on the device in chunks of rows (here forced to
    256 rows per chunk); the result equals the dense select bit for bit."""
    sae, x, meta = workloads.make("C4", T=700, d_sae=32768, device="cuda")
    with _with_paths(False):
        want_v, want_i = ops._topk(sae, x)
    monkeypatch.setattr(ops, "TOPK_REDO_BYTES", 256 * 32768 * 2)
    with _with_paths(True, topk_cap=40):  # most lists overflow
        cnt_over = []
        real = ops.overflow_rows

        def spy(cnt, cap):
            cnt_over.append(int((cnt > cap).sum()))
            return real(cnt, cap)
        monkeypatch.setattr(ops, "overflow_rows", spy)
        got_v, got_i = ops._topk_rows(sae, x)
    assert cnt_over[0] > 512  # the redo spans all three chunks
    assert torch.equal(got_i, want_i) and _bits_equal(got_v, want_v)


def test_topk_row_path_keeps_nan_features():
    """A NaN token (every feature NaN: its list overflows) and a NaN column of W_enc (one NaN
    feature in every row, inside and outside the floor slice) select as the dense top-k does:
    NaN first, by column."""
    sae, x, meta = workloads.make("C4", T=300, d_sae=32768, device="cuda")
    x = x.clone()
    x[11, 7] = float("nan")
    W = sae.W_enc.clone()
    W[:, 20000] = float("nan")
    W[:, 100] = float("nan")
    sae.W_enc = W
    want_v, want_i = ops._topk_dense(sae, x)
    assert bool(torch.isnan(want_v[:, 0]).all())
    got_v, got_i = ops._topk_rows(sae, x)
    assert torch.equal(got_i, want_i) and _bits_equal(got_v, want_v)
    assert int(got_i[0, 0]) == 100 and int(got_i[0, 1]) == 20000


def test_rows_topk_above_1024_with_short_and_nan_rows():
    """rows_topk for k in (1024, 4096]: rows with fewer than k candidates (zero padding at the
    lowest free columns), more than k, and NaN candidates, against topk_rows of the dense rows."""
    g = torch.Generator().manual_seed(11)
    M, N, cap = 6, 8192, 4096
    f = torch.zeros(M, N)
    nz = [1500, 3500, 4096, 1100, 2000, 3000]
    for m, n in enumerate(nz):
        cols = torch.randperm(N, generator=g)[:n]
        f[m, cols] = torch.rand(n, generator=g) + 0.01
    f[1, 5] = float("nan")
    f[4, 4000] = float("nan")
    f[4, 17] = float("nan")
    f = f.to(torch.float16)
    cnt = (f != 0).sum(1).to(torch.int32)  # the planted NaNs may add to a row's count
    assert int(cnt.max()) <= cap
    idx = torch.zeros(M, cap, dtype=torch.int32)
    val = torch.zeros(M, cap, dtype=torch.float16)
    for m in range(M):
        cols = torch.nonzero(f[m] != 0).flatten()
        perm = cols[torch.randperm(cols.numel(), generator=g)]
        idx[m, :cols.numel()] = perm.to(torch.int32)
        val[m, :cols.numel()] = f[m, perm]
    fg = f.cuda()
    for k in (1025, 2000, 4096):
        want_v, want_i = topk_rows(fg, k)
        got_v, got_i = rows_topk(cnt.cuda(), idx.cuda(), val.cuda(), k, N)
        assert torch.equal(got_i, want_i), k
        assert _bits_equal(got_v, want_v), k


def test_topk_encode_sparse_makes_no_host_sync():
    """TopK encode_sparse at C4 width makes no host synchronisation, as the reference's TopK
    branch (ops.py:12-16, 32-36): under torch's sync debug mode "error" any synchronising
    call raises (checked first on a deliberate one)."""
    sae, x, meta = workloads.make("C4", T=1024, device="cuda")
    saeflow_amd.encode_sparse(sae, x)  # first call per shape may time tilings (a sync); not timed here
    torch.cuda.synchronize()
    cnt = torch.ones(4, dtype=torch.int32, device="cuda")
    torch.cuda.set_sync_debug_mode("error")
    try:
        with pytest.raises(RuntimeError):
            int(cnt.max())
        indptr, indices, values = saeflow_amd.encode_sparse(sae, x)
    finally:
        torch.cuda.set_sync_debug_mode("default")
    torch.cuda.synchronize()
    with _with_paths(False):
        want = saeflow_amd.encode_sparse(sae, x)
    assert torch.equal(indices, want[1]) and _bits_equal(values, want[2])
