"""Shared Op flow for the fused gated GELU family.

Behaviour kept from the reference
(examples/TileOPs/tileops/ops/elementwise/gelu_and_mul.py:42-125): ``x`` is
``(M, 2 * N)`` with gate ``x[:, :N]`` and value ``x[:, N:]``; forward makes x
contiguous, validates device / dtype / shape and returns ``(M, N)``;
``eval_roofline`` is ``FLOPS_PER_OUTPUT * M * N`` flops and
``3 * M * N * elem_bytes`` bytes.
"""

from __future__ import annotations

from typing import Dict, Optional

import torch

from tileops.device import get_device_backend
from tileops.kernels.kernel_base import Kernel
from tileops.ops.op_base import Op


class GatedActivationOp(Op):
    _op_name: str = ""
    kernel_cls: type = None
    FLOPS_PER_OUTPUT: int = 0
    _SUPPORTED_DTYPES = (torch.float16, torch.bfloat16, torch.float32)

    def __init__(
        self,
        M: int,
        N: int,
        dtype: torch.dtype,
        *,
        kernel_map: Optional[Dict[str, Kernel]] = None,
    ):
        if dtype not in self._SUPPORTED_DTYPES:
            names = ", ".join(str(dt) for dt in self._SUPPORTED_DTYPES)
            raise ValueError(
                f"{type(self).__name__} does not support dtype {dtype}. Supported: [{names}]"
            )
        self.M = int(M)
        self.N = int(N)
        self.dtype = dtype
        self.output_dtype = dtype
        self.x_shape = (self.M, 2 * self.N)
        self.out_shape = (self.M, self.N)
        self.N_total = self.M * self.N
        self.dispatch_kernel(kernel_map)
        self.kernel = self.kernel_map[self._op_name](self.M, self.N, dtype)

    @property
    def default_kernel_map(self) -> Dict[str, Kernel]:
        return {self._op_name: self.kernel_cls}

    def _validate_input(self, x: torch.Tensor) -> None:
        backend = get_device_backend()
        if not backend.is_device_tensor(x):
            raise ValueError(f"x must be a {backend.name} tensor, got device {x.device}")
        if x.dtype != self.dtype:
            raise ValueError(f"Expected x.dtype {self.dtype}, got {x.dtype}")
        if tuple(x.shape) != self.x_shape:
            raise ValueError(f"Expected x.shape {self.x_shape}, got {tuple(x.shape)}")

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x.contiguous()
        self._validate_input(x)
        return self.kernel(x)

    def eval_roofline(self) -> tuple[int, int]:
        return self.FLOPS_PER_OUTPUT * self.N_total, 3 * self.N_total * self.dtype.itemsize
