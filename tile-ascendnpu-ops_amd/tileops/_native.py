"""ctypes binding of libtileops_hip.so, the C-ABI library of gfx950 kernels.

The declarations mirror include/tileops_hip.h.  Kernel classes call the
``tileops_*`` functions with raw device pointers (``Tensor.data_ptr()``) and
the current HIP stream of the tensors' device, so launches are asynchronous
and ordered with the surrounding PyTorch work.

There is no fallback: if the library is missing, or a tensor is not on a HIP
device, the call raises.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

__all__ = [
    "DTYPE_CODES",
    "LIB_PATH",
    "check",
    "dtype_code",
    "lib",
    "require_device",
    "stream_of",
]

LIB_PATH = Path(
    os.environ.get(
        "TILEOPS_HIP_LIB", str(Path(__file__).resolve().parent / "_native" / "libtileops_hip.so")
    )
)

DTYPE_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_float = ctypes.c_float
_c_p = ctypes.c_void_p

# name -> (restype, argtypes); kept in the order of include/tileops_hip.h
SIGNATURES = {
    "tileops_version": (_c_int, []),
    "tileops_error_string": (ctypes.c_char_p, [_c_int]),
    "tileops_unary_fwd": (
        _c_int,
        [_c_int, _c_p, _c_p, _c_i64, _c_int, _c_float, _c_float, _c_int, _c_p],
    ),
    "tileops_isfp_fwd": (_c_int, [_c_int, _c_p, _c_p, _c_i64, _c_int, _c_p]),
    "tileops_gated_gelu_fwd": (_c_int, [_c_int, _c_p, _c_p, _c_i64, _c_i64, _c_int, _c_p]),
    "tileops_fused_add_layernorm_fwd": (
        _c_int,
        [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_float, _c_int, _c_int, _c_p],
    ),
    "tileops_logsumexp_fwd": (_c_int, [_c_p, _c_p, _c_i64, _c_i64, _c_int, _c_p]),
    "tileops_argreduce_fwd": (_c_int, [_c_p, _c_p, _c_i64, _c_i64, _c_int, _c_int, _c_p]),
    "tileops_mha_fwd": (
        _c_int,
        [
            _c_p, _c_p, _c_p, _c_p, _c_p,
            _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
            _c_int, _c_float, _c_float, _c_int, _c_p,
        ],
    ),
    "tileops_gdn_prefill_fwd": (
        _c_int,
        [
            _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p,
            _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
            _c_float, _c_int, _c_p, ctypes.c_size_t, _c_p,
        ],
    ),
    "tileops_gdn_prefill_workspace_bytes": (
        ctypes.c_size_t,
        [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64],
    ),
    "tileops_gdn_prefill_fwd_ex": (
        _c_int,
        [
            _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p,
            _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
            _c_float, _c_int, _c_i64, _c_p, ctypes.c_size_t, _c_p,
        ],
    ),
    "tileops_gdn_prefill_workspace_bytes_ex": (
        ctypes.c_size_t,
        [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64],
    ),
    "tileops_gdn_prefill_fwd_noalloc": (
        _c_int,
        [
            _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p,
            _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
            _c_float, _c_int, _c_p,
        ],
    ),
    "tileops_bitwise_not_fwd": (_c_int, [_c_p, _c_p, _c_i64, _c_int, _c_p]),
    "tileops_add_fwd": (_c_int, [_c_p, _c_p, _c_p, _c_int, _c_p, _c_p, _c_p, _c_float, _c_int, _c_p]),
    "tileops_lerp_fwd": (
        _c_int,
        [_c_p, _c_p, _c_p, _c_p, _c_int, _c_p, _c_p, _c_p, _c_p, _c_float, _c_int, _c_p],
    ),
    "tileops_gla_decode_fwd": (
        _c_int,
        [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_float,
         _c_int, _c_p],
    ),
    "tileops_gdn_decode_fwd": (
        _c_int,
        [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_float, _c_int, _c_p],
    ),
}

_lib = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """Load libtileops_hip.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.is_file():
                    raise RuntimeError(
                        f"tileops: HIP library not found at {LIB_PATH}; build it with "
                        "`make -C tile-ascendnpu-ops_amd/csrc` (or __graft_entry__.build())"
                    )
                handle = ctypes.CDLL(str(LIB_PATH))
                for name, (restype, argtypes) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype = restype
                    fn.argtypes = argtypes
                _lib = handle
    return _lib


def check(code: int, what: str) -> None:
    """Raise RuntimeError for a nonzero tileops return code."""
    if code != 0:
        msg = lib().tileops_error_string(code)
        raise RuntimeError(f"{what} failed ({code}): {msg.decode() if msg else 'unknown'}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"tileops HIP kernels do not support dtype {dtype}") from None


def require_device(*tensors: torch.Tensor) -> None:
    """Every tensor must live in HIP device memory (there is no host path)."""
    for t in tensors:
        if t is not None and (not t.is_cuda or torch.version.hip is None):
            raise RuntimeError(
                f"tileops HIP kernels need tensors on a ROCm GPU, got device {t.device}"
            )


def stream_of(t: torch.Tensor) -> int:
    """Raw hipStream_t of the current PyTorch stream on ``t``'s device."""
    return torch.cuda.current_stream(t.device).cuda_stream
