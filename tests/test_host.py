"""CPU: the C-ABI library loads and exports every declared entry point; host-side
validation mirrors the reference wrappers (no GPU needed: nothing here reaches a kernel)."""

import ctypes
import re
from pathlib import Path

import pytest
import torch

import saeflow_amd
from saeflow_amd import _lib, workloads
from saeflow_amd.kernels import csr_to_dense, dense_to_csr, fused_encode, sparse_decode, topk_rows

ROOT = Path(__file__).resolve().parents[1]


def declared_functions():
    names = []
    for h in (ROOT / "include").glob("*.h"):
        names += re.findall(r"^\s*(?:SF_API\s+)?(?:const\s+)?\w+\*?\s+\**(sf_\w+)\s*\(", h.read_text(), flags=re.M)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = declared_functions()
    assert declared, "no declarations found in include/*.h"
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"
    assert sorted(_lib.SIGNATURES) == declared, "ctypes signatures out of sync with include/"
    assert lib.sf_abi_version() == _lib.ABI_VERSION


def declared_arity():
    """Parameter count of every sf_* declaration in include/*.h."""
    out = {}
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"\b(sf_\w+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
            params = m.group(2).strip()
            out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_ctypes_signatures_match_the_header_arity():
    """A ctypes signature with a wrong argument count would pass values in the wrong slots:
    every binding in _lib.SIGNATURES has as many arguments as its declaration."""
    arity = declared_arity()
    assert sorted(arity) == sorted(_lib.SIGNATURES)
    for name, (_, args) in _lib.SIGNATURES.items():
        assert len(args) == arity[name], f"{name}: header {arity[name]} parameters, ctypes {len(args)}"


def test_c_abi_rejects_bad_arguments_without_touching_the_gpu():
    lib = _lib.load()
    rc = lib.sf_encode(None, 0, 0, 7, None, 0, 0, 1, None, 1, None, 1, None, 1, None, 0, 0, 1, None, 4, 4, 4, 0,
                       None, None, 0, None)
    assert rc == _lib.SF_EINVAL and b"dtype" in lib.sf_last_error()
    rc = lib.sf_encode(None, 0, 0, 1, None, 0, 0, 1, None, 1, None, 1, None, 1, None, 0, 0, 1, None, 4, 4, 4, 1,
                       None, None, 0, None)
    assert rc == _lib.SF_EINVAL and b"threshold" in lib.sf_last_error()
    for bad_cfg in [(128, 64, 64, 8, 8, 0), (256, 256, 64, 0, 8, 0), (256, 256, 64, 4, 8, -1)]:
        cfg = (ctypes.c_int32 * 6)(*bad_cfg)  # untiled block sizes, GROUP_M < 1, GROUP_N < 0
        rc = lib.sf_encode(1, 4, 1, 1, 1, 4, 1, 1, 1, 1, 1, 1, None, 1, 1, 4, 1, 1, None, 4, 4, 4, 0, cfg, None, 0,
                           None)
        assert rc == _lib.SF_EINVAL and b"tile config" in lib.sf_last_error()
    assert lib.sf_topk(None, 0, 0, 1, 4, 10, 11, None, None, None) == _lib.SF_EINVAL
    assert b"out of range" in lib.sf_last_error()
    # any k <= N is accepted (k above the LDS limit included); here only the NULL buffers fail
    assert lib.sf_topk(None, 0, 0, 1, 4, 5000, 2000, None, None, None) == _lib.SF_EINVAL
    assert b"NULL" in lib.sf_last_error()
    assert lib.sf_rows_topk(None, None, None, 1, 8, 4, 5000, 4097, None, None, None) == _lib.SF_EINVAL
    assert b"maximum" in lib.sf_last_error()
    # decode tile config: both entries must be positive (checked before any launch)
    bad = (ctypes.c_int32 * 2)(0, 128)
    rc = lib.sf_decode(16, 16, 16, 1, 4, 16, 8, 1, 1, 4, None, 0, 16, 8, 1, 1, 1, 8, bad, None)
    assert rc == _lib.SF_EINVAL and b"tile config" in lib.sf_last_error()
    assert lib.sf_compact(None, 0, 0, 1, -1, 4, None, 0, None, None, None) == _lib.SF_EINVAL
    # empty work is a no-op, not an error
    assert lib.sf_encode(None, 0, 0, 1, None, 0, 0, 1, None, 1, None, 1, None, 1, None, 0, 0, 1, None, 0, 8, 8, 0,
                         None, None, 0, None) == _lib.SF_OK
    # row counts are defined for relu / jumprelu only
    rc = lib.sf_encode(16, 64, 1, 1, 16, 64, 1, 1, 16, 1, 16, 1, None, 1, 16, 64, 1, 1, 16, 8, 64, 64, 2, None,
                       16, 1 << 20, None)
    assert rc == _lib.SF_EINVAL and b"relu" in lib.sf_last_error()
    # a missing workspace is rejected before any launch
    rc = lib.sf_encode(16, 64, 1, 1, 16, 64, 1, 1, 16, 1, 16, 1, None, 1, 16, 64, 1, 1, None, 8, 64, 64, 0, None,
                       None, 0, None)
    assert rc == _lib.SF_EINVAL and b"workspace" in lib.sf_last_error()
    nb = ctypes.c_int64()
    assert lib.sf_encode_workspace_size(16384, 2304, 1, ctypes.byref(nb)) == _lib.SF_OK
    assert nb.value == 16384 * 2304 * 2 + 512  # x' and the GEMM's tile counters
    assert lib.sf_encode_workspace_size(3, 50, 0, ctypes.byref(nb)) == _lib.SF_OK
    assert nb.value == (3 * 192 * 4 + 255) // 256 * 256 + 512
    assert lib.sf_last_error() == b""
    got = (ctypes.c_int32 * 6)()
    assert lib.sf_encode_config(16384, 65536, 2304, 1, got) == _lib.SF_OK and list(got) == [256, 256, 64, 1, 8, 8]
    # the allocation-free encode checks its sizes against its fixed array before any HIP call:
    # any number of tokens runs in chunks, but one 256-row block of x' must fit the array
    args = (16, 64, 1, 1, 16, 64, 1, 1, 16, 1, 16, 1, None, 1, 16, 64, 1, 1, None)
    rc = lib.sf_encode_noalloc(*args, 16384, 64, 65664, 0, None, None)  # 256 x 65664 x 2 B > 32 MiB
    assert rc == _lib.SF_EINVAL and b"scratch array" in lib.sf_last_error()
    rc = lib.sf_encode_noalloc(*args, 300, 64, 65664, 0, None, None)  # even for fewer rows than a block
    assert rc == _lib.SF_EINVAL and b"scratch array" in lib.sf_last_error()
    rc = lib.sf_encode_noalloc(*args, 1 << 40, 64, 2304, 0, None, None)  # no overflow in the byte count
    assert rc == _lib.SF_EINVAL and b"too large" in lib.sf_last_error()
    assert lib.sf_encode_noalloc(*args, 0, 64, 2304, 0, None, None) == _lib.SF_OK  # empty: no-op


def test_row_candidate_capacity_bound_is_the_header_one():
    """sf_encode_rows takes 0 <= cap <= 4096 (the lists sf_rows_to_csr and sf_rows_topk read),
    as its declaration says; a larger capacity is rejected before any launch."""
    lib = _lib.load()
    args = (16, 64, 1, 1, 16, 64, 1, 1, 16, 1, 16, 1, None, 1, None, 16, 16, 16, 1)
    for cap in (4097, 1 << 24, -1):
        rc = lib.sf_encode_rows(*args, cap, 8, 64, 64, 0, None, 16, 1 << 20, None)
        assert rc == _lib.SF_EINVAL and b"capacity" in lib.sf_last_error(), cap
    # 4096 itself passes validation: only the NULL-aligned workspace below is wrong
    rc = lib.sf_encode_rows(*args, 4096, 8, 64, 64, 0, None, None, 0, None)
    assert rc == _lib.SF_EINVAL and b"workspace" in lib.sf_last_error()


def test_gathered_entry_points_validate_before_any_launch():
    lib = _lib.load()
    # sf_encode_gather: no row counts, no tile config; NULL row list or count rejected
    rc = lib.sf_encode_gather(16, 64, 1, 1, 8, None, 16, 0, 16, 64, 1, 1, 16, 1, 16, 1, None, 1, 16, 64, 1, 1,
                              8, 64, 64, 0, 16, 1 << 20, None)
    assert rc == _lib.SF_EINVAL and b"NULL row list" in lib.sf_last_error()
    rc = lib.sf_encode_gather(16, 64, 1, 1, 8, 16, 16, -1, 16, 64, 1, 1, 16, 1, 16, 1, None, 1, 16, 64, 1, 1,
                              8, 64, 64, 0, 16, 1 << 20, None)
    assert rc == _lib.SF_EINVAL and b"negative" in lib.sf_last_error()
    assert lib.sf_encode_gather(16, 64, 1, 1, 8, None, None, 0, 16, 64, 1, 1, 16, 1, 16, 1, None, 1, 16, 64, 1, 1,
                                0, 64, 64, 0, None, 0, None) == _lib.SF_OK  # no output rows: no-op
    # sf_topk_gather: k range and NULL row map
    assert lib.sf_topk_gather(None, 0, 0, 1, 4, 10, 11, None, 0, None, 4, None, None, None) == _lib.SF_EINVAL
    assert lib.sf_topk_gather(16, 10, 1, 1, 4, 10, 3, None, 0, None, 4, 16, 16, None) == _lib.SF_EINVAL
    assert b"NULL row list" in lib.sf_last_error()
    assert lib.sf_topk_gather(16, 10, 1, 1, 4, 10, 3, 16, -2, 16, 4, 16, 16, None) == _lib.SF_EINVAL
    # sf_overflow_rows: the count pointer is always written
    assert lib.sf_overflow_rows(None, 8, 4, None, None, None) == _lib.SF_EINVAL
    assert lib.sf_overflow_rows(16, 8, -1, 16, 16, None) == _lib.SF_EINVAL


def test_best_config_is_none_before_a_tuned_launch():
    from saeflow_amd.kernels import best_config
    from saeflow_amd.kernels import encode as kenc
    assert kenc._last_config is None and best_config() is None  # encode.py:142-144


def test_python_validation_matches_reference_errors():
    x, W = torch.randn(3, 4), torch.randn(4, 6)
    b_enc, b_dec = torch.zeros(6), torch.zeros(4)
    with pytest.raises(ValueError, match="supports"):
        fused_encode(x, W, b_enc, b_dec, activation="gelu")
    with pytest.raises(ValueError, match="threshold"):
        fused_encode(x, W, b_enc, b_dec, activation="jumprelu")
    with pytest.raises(ValueError, match="d_in"):
        fused_encode(torch.randn(3, 5), W, b_enc, b_dec)
    with pytest.raises(ValueError, match="GPU"):
        fused_encode(x, W, b_enc, b_dec)  # CPU tensors: no CPU path, loud failure
    with pytest.raises(ValueError, match="GPU"):
        dense_to_csr(torch.zeros(2, 3))
    with pytest.raises(RuntimeError, match="out of range"):
        topk_rows(torch.zeros(2, 3), 4)
    with pytest.raises(ValueError, match="activation"):
        saeflow_amd.SAE(4, 8, "gelu")
    with pytest.raises(ValueError, match="needs k"):
        saeflow_amd.SAE(4, 8, "topk")


def test_empty_batches_return_empty_outputs():
    out = fused_encode(torch.zeros(0, 4), torch.zeros(4, 6), torch.zeros(6), torch.zeros(4))
    assert out.shape == (0, 6)
    out = sparse_decode(torch.zeros(1, dtype=torch.int64), torch.zeros(0, dtype=torch.int32), torch.zeros(0),
                        torch.zeros(6, 4))
    assert out.shape == (0, 4)
    assert csr_to_dense(torch.zeros(1, dtype=torch.int64), torch.zeros(0, dtype=torch.int32), torch.zeros(0),
                        7).shape == (0, 7)


def test_sae_container_matches_reference_init():
    torch.manual_seed(0)
    sae = saeflow_amd.SAE(16, 40, "jumprelu")
    assert sae.W_enc.shape == (16, 40) and sae.W_dec.shape == (40, 16)
    torch.testing.assert_close(sae.W_dec.norm(dim=1), torch.ones(40))
    assert torch.equal(sae.W_enc, sae.W_dec.T)
    assert sae.threshold.shape == (40,) and not sae.W_enc.requires_grad
    assert saeflow_amd.SAE(16, 40).threshold is None


def test_workload_recipe():
    sae, x, meta = workloads.make("C3", T=512, d_sae=8192)
    assert sae.W_enc.dtype == torch.bfloat16 and x.shape == (512, 2304)
    torch.testing.assert_close(sae.W_dec.float().norm(dim=1), torch.ones(8192), atol=1e-2, rtol=0)
    assert abs(meta["l0_expected"] - 64 * 8192 / 65536) <= 0.5
    pre = (x.float() - sae.b_dec.float()) @ sae.W_enc.float()
    assert 0.9 < pre.std().item() < 1.1
    l0 = ((pre > sae.threshold.float()) & (pre > 0)).sum(1).float().mean().item()
    assert abs(l0 - meta["l0_expected"]) < 2.0
    sae1, _, _ = workloads.make("C1", T=256, d_sae=4096)
    assert sae1.W_enc.dtype == torch.float32 and float(sae1.b_enc[0]) == pytest.approx(-2.8)
    # same seed -> identical tensors
    sae2, x2, _ = workloads.make("C3", T=512, d_sae=8192)
    assert torch.equal(x, x2) and torch.equal(sae.threshold, sae2.threshold)


def test_backward_c_abi_rejects_bad_arguments_without_touching_the_gpu():
    """The backward entry points check every argument before their first launch, and the
    host-side bounds follow their documented formulas (C3: d_in 2304 bf16, d_sae 65536,
    nnz 1052702)."""
    lib = _lib.load()
    EINVAL, P = _lib.SF_EINVAL, 16  # P: a non-null stand-in pointer, never dereferenced here
    mi, ms, wf = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    assert lib.sf_backward_bounds(65536, 1052702, 2304, 1, ctypes.byref(mi), ctypes.byref(ms), ctypes.byref(wf)) == 0
    # items: one per used feature (at most min(N, nnz)) plus one per 256 further entries
    # slots: a feature of n > 64 entries has ceil(n / 256) <= n / 65 of them
    assert (mi.value, ms.value) == (65536 + 1052702 // 256 + 1, 1052702 // 65 + 1)
    assert wf.value == (5 + 1) * 1052702  # 288 16-B chunks a row = 5 slabs of 64, then the CSC-order copy
    assert lib.sf_backward_bounds(10, 100, 64, 7, ctypes.byref(mi), ctypes.byref(ms), ctypes.byref(wf)) == EINVAL
    cols = lambda **kw: lib.sf_backward_columns(*[kw.get(k, v) for k, v in (
        ("colptr", P), ("csc_row", P), ("csc_pos", P), ("plan", P), ("item_col", P), ("multi_col", P),
        ("slot_item", P), ("max_items", 10), ("max_slots", 3), ("values", P), ("val_dt", 1), ("g_val", None), ("gval_dt", 0),
        ("w_dec", P), ("sw", 64), ("xs", P), ("sx", 64), ("g_xhat", P), ("sg", 64), ("dt", 1), ("N", 10),
        ("M", 4), ("D", 64), ("nnz", 100), ("g_pre", P), ("d_wdec", P), ("d_wenc", P), ("d_benc", P),
        ("partials", P), ("work", P), ("work_floats", 200), ("stream", None))])
    assert cols(dt=7) == EINVAL and b"dtype" in lib.sf_last_error()
    assert cols(N=-1) == EINVAL and b"negative" in lib.sf_last_error()
    assert cols(work_floats=10) == EINVAL and b"work of" in lib.sf_last_error()
    assert cols(partials=None) == EINVAL and b"NULL" in lib.sf_last_error()
    assert cols(g_pre=None) == EINVAL and b"g_pre" in lib.sf_last_error()
    assert cols(slot_item=None) == EINVAL and b"NULL" in lib.sf_last_error()
    assert cols(d_wenc=None) == EINVAL and b"NULL" in lib.sf_last_error()
    nb = ctypes.c_int64()
    big = (1 << 23) + 1  # past the counting sort: atomic placement, 2^18 rows at most
    assert lib.sf_csr_transpose_workspace_size(100, big, 50, ctypes.byref(nb)) == 0
    assert nb.value == 4 * (big + 2 * 50) + 256
    assert lib.sf_csr_transpose(P, P, (1 << 18) + 1, big, 50, P, P, P, P, 1 << 40, None) == EINVAL
    assert b"2^18" in lib.sf_last_error()
    assert lib.sf_csr_transpose(P, P, -1, 10, 0, P, P, P, P, 0, None) == EINVAL
    assert lib.sf_backward_plan(P, -1, 0, P, P, P, P, None) == EINVAL
    assert lib.sf_backward_plan(P, 10, 0, P, P, P, None, None) == EINVAL and b"NULL" in lib.sf_last_error()
    assert lib.sf_shifted_input(P, 64, 1, 9, P, 1, 4, 64, 1, P, None) == EINVAL
    assert lib.sf_transpose(P, 4, 64, 64, 9, None, P, None) == EINVAL
    assert lib.sf_transpose(P, 4, 64 * 65536, 64 * 65536, 1, None, P, None) == EINVAL
    assert lib.sf_column_sums(P, -1, 8, 8, 1, 1.0, 0, P, P, 64, None) == EINVAL
    assert lib.sf_matvec(P, -1, 8, 8, 1, 1, P, 1.0, 0, P, P, 64, None) == EINVAL
    assert lib.sf_matvec(P, 8, 8, 8, 1, 1, P, 1.0, 0, P, P, 1, None) == EINVAL  # workspace too small
