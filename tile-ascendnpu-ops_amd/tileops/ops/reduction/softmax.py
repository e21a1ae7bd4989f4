"""LogSumExpFwdOp: y = logsumexp(x, dim, keepdim) in the input dtype.

Reference: examples/TileOPs/tileops/ops/reduction/softmax.py:36-218 (dtype
float32 / float16 / bfloat16, int or list dim, roofline ``4 * M * N`` flops and
``(M * N + M) * elem_bytes`` bytes).
"""

from __future__ import annotations

from math import prod
from typing import Dict, List, Optional, Tuple, Union

import torch

from tileops.device import get_device_backend
from tileops.kernels.kernel_base import Kernel
from tileops.kernels.reduction.logsumexp.logsumexp import LogSumExpKernel
from tileops.ops._multidim import (
    EmptyDimPolicy,
    flatten_for_multidim,
    normalize_dim,
    restore_multidim_shape,
)
from tileops.ops.op_base import Op

__all__ = ["LogSumExpFwdOp"]


class LogSumExpFwdOp(Op):
    """LogSumExp along ``dim`` (int or list of ints).

    Args:
        dtype: float32, float16 or bfloat16.
        dim: Reduction dim(s) (default -1).
        keepdim: Keep reduced dims as size 1.
        kernel_map: Optional kernel override.
    """

    _op_kind = "logsumexp"
    _kernel_key = "logsumexp_fwd"
    _kernel_class = LogSumExpKernel
    _supports_multidim = True
    _empty_dim_policy: EmptyDimPolicy = "reject"
    _static_axes: frozenset = frozenset()

    def __init__(
        self,
        dtype: torch.dtype,
        dim: Union[int, List[int]] = -1,
        keepdim: bool = False,
        *,
        kernel_map: Optional[Dict[str, Kernel]] = None,
    ):
        self.dtype = dtype
        self._committed_dtype = dtype
        self.dim = dim
        self.N: Optional[int] = None
        self.keepdim = keepdim
        self.dispatch_kernel(kernel_map)
        self._kernel_cache: Dict[tuple, object] = {}
        self.kernel: object | None = None
        self._last_roofline_spec: tuple[int, int, torch.dtype] | None = None

    @property
    def default_kernel_map(self) -> Dict[str, Kernel]:
        return {self._kernel_key: self._kernel_class}

    def _validate(self, x: torch.Tensor) -> None:
        backend = get_device_backend()
        if not backend.is_device_tensor(x):
            raise ValueError(f"x must be a {backend.name} tensor, got device {x.device}")
        if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise ValueError(f"x.dtype must be float16, bfloat16, or float32, got {x.dtype}")
        if self._committed_dtype is not None and x.dtype != self._committed_dtype:
            raise ValueError(f"Expected x.dtype {self._committed_dtype}, got {x.dtype}")
        if x.ndim == 0:
            raise ValueError("Input tensor must be at least 1D")
        self.dtype = x.dtype

    def _get_or_create_kernel(self, M: int, N: int, dtype: torch.dtype, device_index=None):
        key = (M, N, dtype, device_index)
        if key not in self._kernel_cache:
            self._kernel_cache[key] = self.kernel_map[self._kernel_key](
                M, N, self._op_kind, dtype, device_index=device_index
            )
        return self._kernel_cache[key]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        self._validate(x)
        orig_shape = x.shape
        dim = self.dim
        if isinstance(dim, (list, tuple)) or dim is None:
            dims = normalize_dim(dim, x.ndim, empty_dim_policy=self._empty_dim_policy)
            self._static_axes = frozenset([(0, d) for d in dims])
            x, orig_shape, _ = flatten_for_multidim(x, dims)
            N = x.shape[-1]
            M = prod(x.shape[:-1])
            self._last_roofline_spec = (M, N, x.dtype)
            kernel = self._get_or_create_kernel(M, N, x.dtype, x.device.index)
            self.kernel = kernel
            y = kernel(x.reshape(M, N))
            return restore_multidim_shape(y, orig_shape, dims, self.keepdim)

        if dim < -x.ndim or dim >= x.ndim:
            raise IndexError(
                f"Dimension out of range (expected to be in range of "
                f"[{-x.ndim}, {x.ndim - 1}], but got {dim})"
            )
        d = dim % x.ndim
        N = x.shape[d]
        if self.N is not None and N != self.N:
            raise ValueError(
                f"{type(self).__name__}: committed N={self.N} does not match "
                f"x.shape[{dim}]={N}"
            )
        self._static_axes = frozenset({(0, d)})
        M = prod([s for i, s in enumerate(x.shape) if i != d])
        self._last_roofline_spec = (M, N, x.dtype)
        moved = d != x.ndim - 1
        if moved:
            x = x.movedim(d, -1)
        x = x.contiguous().reshape(M, N)
        kernel = self._get_or_create_kernel(M, N, x.dtype, x.device.index)
        self.kernel = kernel
        y = kernel(x)
        if self.keepdim:
            shape = list(orig_shape)
            shape[d] = 1
            return y.reshape(shape)
        shape = [s for i, s in enumerate(orig_shape) if i != d]
        return y.squeeze() if not shape else y.reshape(shape)

    def eval_roofline(self) -> tuple[int, int]:
        if self._last_roofline_spec is None:
            raise RuntimeError(
                f"{type(self).__name__}.eval_roofline() requires a prior forward() "
                "call to bind dynamic input shape"
            )
        M, N, dtype = self._last_roofline_spec
        return 4 * M * N, (M * N + M) * dtype.itemsize
