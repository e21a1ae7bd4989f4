"""Shared base of the reduce Ops (dim handling, reshapes, kernel cache, roofline).

Behaviour kept from the reference's ``_ReduceOpBase``
(examples/TileOPs/tileops/ops/reduction/reduce.py:65-519): ``dim`` may be an
int, a list/tuple of ints or ``None`` (full reduction, flattened index space);
the input is validated (device, dtype, ``ndim >= 1``), the reduced dim is
moved last and flattened to ``(M, N)``, kernels are cached per ``(M, N)``, and
the ``(M,)`` result is reshaped for ``keepdim``.  The gfx950 kernels accept
any ``N`` directly, so no host-side alignment padding is ever applied.
"""

from math import prod
from typing import Dict, List, Optional, Tuple, Union

import torch

from tileops.device import get_device_backend
from tileops.kernels.kernel_base import Kernel
from tileops.ops._multidim import (
    EmptyDimPolicy,
    flatten_for_multidim,
    normalize_dim,
    restore_multidim_shape,
)
from tileops.ops.op_base import Op

__all__ = ["_ReduceOpBase"]


class _ReduceOpBase(Op):
    """Common base for reduce ops; subclasses set ``_op_kind``, ``_kernel_key``,
    ``_kernel_cls`` and may override ``_validate_dim``."""

    _op_kind: str = ""
    _kernel_key: str = "reduce"
    _kernel_cls: type = None
    _kernel_handles_padding: bool = True
    _empty_dim_policy: EmptyDimPolicy = "reject"

    def __init__(
        self,
        dtype: torch.dtype,
        dim: Union[int, List[int], Tuple[int, ...], None] = None,
        keepdim: bool = False,
        *,
        kernel_map: Optional[Dict[str, Kernel]] = None,
    ):
        self.dtype = dtype
        self.dim = dim
        self.keepdim = keepdim
        self._validate_dim()
        self.dispatch_kernel(kernel_map)
        self._kernel_cache: Dict[tuple, object] = {}
        self._last_roofline_mn: Optional[tuple[int, int]] = None

    def _validate_dim(self) -> None:
        dim = self.dim
        if isinstance(dim, bool):
            raise TypeError(
                f"dim must not be bool (subclasses int but is not a valid axis), got {dim!r}"
            )
        if dim is None or isinstance(dim, int):
            return
        if isinstance(dim, (list, tuple)):
            for d in dim:
                if isinstance(d, bool) or not isinstance(d, int):
                    raise TypeError(f"All elements of dim must be int (not bool), got {dim!r}")
            return
        raise TypeError(
            f"dim must be int, list[int], tuple[int, ...], or None, got {type(dim).__name__}"
        )

    @property
    def default_kernel_map(self) -> Dict[str, Kernel]:
        return {self._kernel_key: self._kernel_cls}

    def _build_kernel_kwargs(self) -> dict:
        return {}

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x2d, orig_shape, dim_info, kernel = self._prepare_input(x)
        y = kernel(x2d)
        return self._reshape_output(y, orig_shape, dim_info)

    def _validate_input_tensor(self, x: torch.Tensor) -> None:
        backend = get_device_backend()
        if not backend.is_device_tensor(x):
            raise ValueError(f"x must be a {backend.name} tensor")
        if x.dtype != self.dtype:
            raise ValueError(f"Expected x.dtype {self.dtype}, got {x.dtype}")
        if x.ndim == 0:
            raise ValueError("Input tensor must be at least 1D")

    def eval_roofline(self) -> tuple[int, int]:
        if self._last_roofline_mn is None:
            raise RuntimeError(
                f"{type(self).__name__}.eval_roofline() requires a prior forward() "
                "call to bind dynamic input shape"
            )
        M, N = self._last_roofline_mn
        elem = self.dtype.itemsize
        if self._op_kind in {"argmax", "argmin"}:
            return M * N, M * N * elem + M * 8
        return M * N, (M * N + M) * elem

    def _get_or_create_kernel(self, M: int, N: int) -> object:
        key = (M, N)
        if key not in self._kernel_cache:
            self._kernel_cache[key] = self.kernel_map[self._kernel_key](
                M, N, self._op_kind, self.dtype, **self._build_kernel_kwargs()
            )
        return self._kernel_cache[key]

    def _prepare_input(self, x: torch.Tensor):
        self._validate_input_tensor(x)
        orig_shape = x.shape
        if isinstance(self.dim, (list, tuple)) or self.dim is None:
            dims = normalize_dim(self.dim, x.ndim, empty_dim_policy=self._empty_dim_policy)
            x, orig_shape, _ = flatten_for_multidim(x, dims)
            N = x.shape[-1]
            M = prod(x.shape[:-1])
            self._last_roofline_mn = (M, N)
            return x.reshape(M, N), orig_shape, dims, self._get_or_create_kernel(M, N)
        if self.dim < -x.ndim or self.dim >= x.ndim:
            raise IndexError(
                f"Dimension out of range (expected to be in range of "
                f"[{-x.ndim}, {x.ndim - 1}], but got {self.dim})"
            )
        dim = self.dim % x.ndim
        N = x.shape[dim]
        M = prod([s for i, s in enumerate(x.shape) if i != dim])
        self._last_roofline_mn = (M, N)
        if dim != x.ndim - 1:
            x = x.movedim(dim, -1)
        x = x.contiguous().reshape(M, N)
        return x, orig_shape, dim, self._get_or_create_kernel(M, N)

    def _reshape_output(self, y: torch.Tensor, orig_shape: torch.Size, dim_info) -> torch.Tensor:
        if isinstance(dim_info, list):
            return restore_multidim_shape(y, orig_shape, dim_info, self.keepdim)
        dim = dim_info
        if self.keepdim:
            shape = list(orig_shape)
            shape[dim] = 1
            return y.reshape(shape)
        shape = [s for i, s in enumerate(orig_shape) if i != dim]
        return y.squeeze() if not shape else y.reshape(shape)
