"""Shared Op flow for the flat elementwise family.

Behaviour kept from the reference Ops (e.g.
examples/TileOPs/tileops/ops/elementwise/hardswish.py:27-107,
examples/TileOPs/tileops/ops/elementwise/isnan.py:36-115): validate device /
dtype / element count, flatten with ``contiguous().reshape(-1)``, run the
kernel, reshape back; ``eval_roofline`` is ``FLOPS_PER_ELEM * N`` flops and
``N * (in_bytes + out_bytes)`` bytes.
"""

from __future__ import annotations

from typing import Dict, Optional

import torch

from tileops.device import get_device_backend
from tileops.kernels.kernel_base import Kernel
from tileops.ops.op_base import Op


class FlatElementwiseOp(Op):
    """Single-input, single-output op over ``N_total`` flattened elements."""

    _op_name: str = ""
    kernel_cls: type = None
    FLOPS_PER_ELEM: int = 1

    @property
    def default_kernel_map(self) -> Dict[str, Kernel]:
        return {self._op_name: self.kernel_cls}

    def _validate_input(self, input: torch.Tensor) -> None:
        backend = get_device_backend()
        if not backend.is_device_tensor(input):
            raise ValueError(f"input must be a {backend.name} tensor, got device {input.device}")
        if input.dtype != self.dtype:
            raise ValueError(f"Expected input.dtype {self.dtype}, got {input.dtype}")
        if input.numel() != self.N_total:
            raise ValueError(f"Expected {self.N_total} elements, got {input.numel()}")

    def _eager_forward(self, input: torch.Tensor) -> torch.Tensor:
        orig_shape = input.shape
        flat = input.contiguous().reshape(-1)
        return self.kernel(flat).reshape(orig_shape)

    def forward(self, input: torch.Tensor) -> torch.Tensor:
        self._validate_input(input)
        return self._eager_forward(input)

    @property
    def total_memory(self) -> float:
        """Read x + write y."""
        return self.N_total * (self.dtype.itemsize + self.output_dtype.itemsize)

    def eval_roofline(self) -> tuple[int, int]:
        return self.FLOPS_PER_ELEM * self.N_total, int(self.total_memory)


class InplaceActivationOp(FlatElementwiseOp):
    """Activation with the reference's ``inplace`` flag (Hardswish / Hardsigmoid)."""

    def __init__(
        self,
        N_total: int,
        dtype: torch.dtype,
        inplace: bool = False,
        *,
        kernel_map: Optional[Dict[str, Kernel]] = None,
    ):
        self.N_total = N_total
        self.dtype = dtype
        self.inplace = inplace
        self.output_dtype = dtype
        self.dispatch_kernel(kernel_map)
        self.kernel = self.kernel_map[self._op_name](N_total, dtype)

    def forward(self, input: torch.Tensor) -> torch.Tensor:
        self._validate_input(input)
        if self.inplace:
            if input.is_contiguous():
                # the kernel writes each element over the one it read: no
                # second buffer and no copy back
                flat = input.reshape(-1)
                self.kernel(flat, out=flat)
                return input
            result = self._eager_forward(input)
            input.copy_(result.reshape(input.shape))
            return input
        return self._eager_forward(input)


class PredicateOp(FlatElementwiseOp):
    """Float predicate with bool output (Isnan / Isinf / Isfinite)."""

    _SUPPORTED_DTYPES = (torch.float16, torch.bfloat16, torch.float32)

    def __init__(
        self,
        N_total: int,
        dtype: torch.dtype,
        *,
        kernel_map: Optional[Dict[str, Kernel]] = None,
    ):
        if dtype not in self._SUPPORTED_DTYPES:
            names = ", ".join(str(dt) for dt in self._SUPPORTED_DTYPES)
            raise ValueError(
                f"{type(self).__name__} does not support dtype {dtype}. Supported: [{names}]"
            )
        self.N_total = N_total
        self.dtype = dtype
        self.output_dtype = torch.bool
        self.dispatch_kernel(kernel_map)
        self.kernel = self.kernel_map[self._op_name](N_total, dtype)
