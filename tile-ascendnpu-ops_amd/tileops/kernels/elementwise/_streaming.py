"""Shared Kernel classes for the streaming elementwise family.

One implementation per C-ABI entry point; the per-op modules
(``hardswish``, ``hardsigmoid``, ``clamp_scalar``, ``isnan`` ...) bind the
reference's class names to it.  Constructor signatures, attributes and error
messages follow the reference Kernel classes, e.g.
examples/TileOPs/tileops/kernels/elementwise/hardswish/hardswish.py:82-156 and
examples/TileOPs/tileops/kernels/elementwise/isnan/isnan.py:75-156.
"""

from __future__ import annotations

from typing import Optional

import torch

from tileops import _native
from tileops.kernels.kernel_base import Kernel

_FLOAT_DTYPES = (torch.float16, torch.bfloat16, torch.float32)

# enum tileops_unary_op / tileops_predicate (include/tileops_hip.h)
HARDSWISH, HARDSIGMOID, CLAMP, MISH = 0, 1, 2, 3
ISNAN, ISINF, ISFINITE = 0, 1, 2
CLAMP_HAS_MIN, CLAMP_HAS_MAX = 1, 2


def _check_dtype(cls: type, dtype: torch.dtype, supported: tuple) -> None:
    if dtype not in supported:
        names = ", ".join(str(dt) for dt in supported)
        raise ValueError(f"{cls.__name__} only supports dtypes [{names}], got {dtype}")


class UnaryFwdKernel(Kernel):
    """y = f(x) over a flat vector of ``N_total`` elements (fp32 opmath)."""

    SUPPORTED_DTYPES = _FLOAT_DTYPES
    _unary_op: int = -1
    profile_kernel_name = r"tileops(?:::|\d+)unary_(vec|scalar)_kernel"

    def __init__(self, N_total: int, dtype: torch.dtype, config: Optional[dict] = None):
        super().__init__()
        _check_dtype(type(self), dtype, self.SUPPORTED_DTYPES)
        self.N_total = int(N_total)
        self.dtype = dtype
        self.output_dtype = dtype
        self.init_config(config)

    @property
    def default_config(self) -> dict:
        # unary_vec_kernel: 256-thread workgroups, one 16-byte non-temporal
        # pack per thread, a grid covering the whole tensor
        return {"threads": 256, "vector_bytes": 16, "packs_per_thread": 1}

    def _bounds(self) -> tuple[float, float, int]:
        return 0.0, 0.0, 0

    def forward(self, x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """``out`` (contiguous, same dtype and size) receives the result; it
        may be ``x`` itself: every element is read before it is written by
        the same thread, so the kernel runs in place."""
        _native.require_device(x)
        self.check_tensor("x", x, dtype=self.dtype, numel=self.N_total)
        x = x.contiguous()
        if out is None:
            y = torch.empty_like(x)
        else:
            self.check_tensor("out", out, dtype=self.dtype, numel=self.N_total)
            if not out.is_contiguous():
                raise ValueError(f"{type(self).__name__}: out must be contiguous")
            y = out
        lo, hi, flags = self._bounds()
        code = _native.lib().tileops_unary_fwd(
            self._unary_op,
            x.data_ptr(),
            y.data_ptr(),
            self.N_total,
            _native.dtype_code(self.dtype),
            lo,
            hi,
            flags,
            _native.stream_of(x),
        )
        _native.check(code, type(self).__name__)
        return y


class PredicateFwdKernel(Kernel):
    """y = pred(x) as torch.bool over a flat vector of ``N_total`` elements."""

    SUPPORTED_DTYPES = _FLOAT_DTYPES
    _predicate: int = -1
    profile_kernel_name = r"tileops(?:::|\d+)isfp_(vec|scalar)_kernel"

    def __init__(self, N_total: int, dtype: torch.dtype, config: Optional[dict] = None):
        super().__init__()
        _check_dtype(type(self), dtype, self.SUPPORTED_DTYPES)
        self.N_total = int(N_total)
        self.dtype = dtype
        self.output_dtype = torch.bool
        self.init_config(config)

    @property
    def default_config(self) -> dict:
        # isfp_vec_kernel: 256-thread workgroups, two 16-byte input packs per
        # thread (256 packs apart), each giving a 4- or 8-byte bool store
        return {"threads": 256, "vector_bytes": 16, "packs_per_thread": 2}

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        _native.require_device(x)
        self.check_tensor("x", x, dtype=self.dtype, numel=self.N_total)
        x = x.contiguous()
        y = torch.empty(x.shape, dtype=torch.bool, device=x.device)
        code = _native.lib().tileops_isfp_fwd(
            self._predicate,
            x.data_ptr(),
            y.data_ptr(),
            self.N_total,
            _native.dtype_code(self.dtype),
            _native.stream_of(x),
        )
        _native.check(code, type(self).__name__)
        return y


class GatedGeluFwdKernel(Kernel):
    """y[M, N] = gelu(x[:, :N]) * x[:, N:] for x[M, 2N] (fp32 opmath)."""

    SUPPORTED_DTYPES = _FLOAT_DTYPES
    _approx: int = 0
    profile_kernel_name = r"tileops(?:::|\d+)gated_gelu_(vec|rows|scalar)_kernel"

    def __init__(self, M: int, N: int, dtype: torch.dtype, config: Optional[dict] = None):
        super().__init__()
        _check_dtype(type(self), dtype, self.SUPPORTED_DTYPES)
        self.M = int(M)
        self.N = int(N)
        self.dtype = dtype
        self.output_dtype = dtype
        self.init_config(config)

    @property
    def default_config(self) -> dict:
        # gated_gelu_vec_kernel: one-shot grid of 256-thread workgroups over
        # the flattened output, one 16-byte gate pack, one value pack and
        # one output pack per thread
        return {"threads": 256, "vector_bytes": 16, "packs_per_thread": 1}

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        _native.require_device(x)
        self.check_tensor("x", x, dtype=self.dtype, shape=(self.M, 2 * self.N))
        x = x.contiguous()
        y = torch.empty((self.M, self.N), dtype=self.dtype, device=x.device)
        code = _native.lib().tileops_gated_gelu_fwd(
            self._approx,
            x.data_ptr(),
            y.data_ptr(),
            self.M,
            self.N,
            _native.dtype_code(self.dtype),
            _native.stream_of(x),
        )
        _native.check(code, type(self).__name__)
        return y
