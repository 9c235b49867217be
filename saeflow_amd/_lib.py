"""ctypes binding of libsaeflow_hip.so (declared in include/saeflow_hip.h).

The library is loaded after torch so that it binds to the HIP runtime torch already
loaded (both name their runtime libamdhip64.so.7): device pointers and streams handed
over from torch tensors then belong to the same runtime. There is no fallback: without
the built library, or with tensors that are not on a ROCm device, every op raises.
"""

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libsaeflow_hip.so"
ABI_VERSION = 4

SF_OK, SF_EINVAL, SF_EHIP, SF_EUNSUPPORTED = 0, 1, 2, 3
ACT = {"relu": 0, "jumprelu": 1, "none": 2}
DTYPE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}

_P, _I64, _I32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int

# argument types of every exported function, in header order
SIGNATURES = {
    "sf_abi_version": (_I32, []),
    "sf_last_error": (ctypes.c_char_p, []),
    "sf_encode": (_I32, [_P, _I64, _I64, _I32, _P, _I64, _I64, _I32, _P, _I32, _P, _I32, _P, _I32,
                         _P, _I64, _I64, _I32, _P, _I64, _I64, _I64, _I32, _P, _P, _I64, _P]),
    "sf_encode_noalloc": (_I32, [_P, _I64, _I64, _I32, _P, _I64, _I64, _I32, _P, _I32, _P, _I32, _P, _I32,
                                 _P, _I64, _I64, _I32, _P, _I64, _I64, _I64, _I32, _P, _P]),
    "sf_encode_workspace_size": (_I32, [_I64, _I64, _I32, _P]),
    "sf_encode_config": (_I32, [_I64, _I64, _I64, _I32, _P]),
    "sf_encode_rows": (_I32, [_P, _I64, _I64, _I32, _P, _I64, _I64, _I32, _P, _I32, _P, _I32, _P, _I32, _P,
                              _P, _P, _P, _I32, _I64, _I64, _I64, _I64, _I32, _P, _P, _I64, _P]),
    "sf_overflow_rows": (_I32, [_P, _I64, _I64, _P, _P, _P]),
    "sf_encode_gather": (_I32, [_P, _I64, _I64, _I32, _I64, _P, _P, _I64, _P, _I64, _I64, _I32, _P, _I32, _P, _I32,
                                _P, _I32, _P, _I64, _I64, _I32, _I64, _I64, _I64, _I32, _P, _I64, _P]),
    "sf_rows_to_csr": (_I32, [_P, _P, _P, _I32, _I64, _I64, _P, _I64, _P, _P, _P]),
    "sf_rows_topk": (_I32, [_P, _P, _P, _I32, _I64, _I64, _I64, _I64, _P, _P, _P]),
    "sf_count_nonzero": (_I32, [_P, _I64, _I64, _I32, _I64, _I64, _P, _P]),
    "sf_scan_counts": (_I32, [_P, _I64, _P, _P]),
    "sf_compact": (_I32, [_P, _I64, _I64, _I32, _I64, _I64, _P, _I64, _P, _P, _P]),
    "sf_decode": (_I32, [_P, _P, _P, _I32, _I64, _P, _I64, _I64, _I32, _I64, _P, _I32, _P, _I64, _I64,
                         _I32, _I64, _I64, _P, _P]),
    "sf_topk": (_I32, [_P, _I64, _I64, _I32, _I64, _I64, _I64, _P, _P, _P]),
    "sf_topk_gather": (_I32, [_P, _I64, _I64, _I32, _I64, _I64, _I64, _P, _I64, _P, _I64, _P, _P, _P]),
    "sf_csr_to_dense": (_I32, [_P, _I64, _P, _P, _I32, _I64, _I64, _I64, _P, _I64, _I32, _P]),
    "sf_csr_transpose_workspace_size": (_I32, [_I64, _I64, _I64, _P]),
    "sf_csr_transpose": (_I32, [_P, _P, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _P]),
    "sf_shifted_input": (_I32, [_P, _I64, _I64, _I32, _P, _I32, _I64, _I64, _I32, _P, _P]),
    "sf_backward_bounds": (_I32, [_I64, _I64, _I64, _I32, _P, _P, _P]),
    "sf_backward_plan": (_I32, [_P, _I64, _I64, _P, _P, _P, _P, _P]),
    "sf_backward_columns": (_I32, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _P, _I32, _P, _I32, _P, _I64, _P, _I64,
                                   _P, _I64, _I32, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _I64, _P]),
    "sf_transpose": (_I32, [_P, _I64, _I64, _I64, _I32, _P, _P, _P]),
    "sf_column_sums": (_I32, [_P, _I64, _I64, _I64, _I32, ctypes.c_float, _I32, _P, _P, _I64, _P]),
    "sf_matvec": (_I32, [_P, _I64, _I64, _I64, _I64, _I32, _P, ctypes.c_float, _I32, _P, _P, _I64, _P]),
}

_lib = None
_lock = threading.Lock()


def load():
    """The loaded library (loads it on first use; raises RuntimeError if it is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is not built: run `python -m saeflow_amd.build` (or __graft_entry__.build())"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype, fn.argtypes = res, args
            if lib.sf_abi_version() != ABI_VERSION:
                raise RuntimeError(f"{LIB_PATH}: ABI {lib.sf_abi_version()} != expected {ABI_VERSION}; rebuild it")
            _lib = lib
    return _lib


def check(rc):
    """Raise for a nonzero sf_status: ValueError for rejected arguments, RuntimeError otherwise."""
    if rc == SF_OK:
        return
    msg = load().sf_last_error().decode(errors="replace")
    raise (ValueError if rc == SF_EINVAL else RuntimeError)(msg)


def dtype_code(t, what):
    try:
        return DTYPE[t.dtype]
    except KeyError:
        raise ValueError(f"{what} has dtype {t.dtype}; supported: float32, bfloat16, float16") from None


def ptr(t):
    return None if t is None else t.data_ptr()


def require_gpu(*named):
    """All given tensors must live on one ROCm (torch 'cuda') device; returns that device."""
    dev = None
    for name, t in named:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError(
                f"{name} is on {t.device}: saeflow_amd runs on the GPU only (HIP kernels for gfx950, no CPU path)"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"{name} is on {t.device}, expected {dev}")
    return dev


def stream(device):
    """torch's current stream on `device`, as the hipStream_t handle the C ABI takes."""
    return torch.cuda.current_stream(device).cuda_stream
