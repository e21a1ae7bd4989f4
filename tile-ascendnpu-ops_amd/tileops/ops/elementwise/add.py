"""AddFwdOp: y = input + alpha * other with PyTorch broadcasting.

Reference: examples/TileOPs/tileops/ops/elementwise/add.py:61-155
(constructor ``(*, input: shape, other: shape, dtype, alpha=1)``,
float dtypes, the rejection message "AddFwdOp does not support dtype ...",
``out_shape = broadcast_shapes(input, other)``; roofline flops
``(1 if alpha == 1 else 2) * N``, bytes ``3 * N * elem_bytes`` with N the
broadcast element count).
"""

from math import prod
from typing import Dict, Optional

import torch

from tileops.device import get_device_backend
from tileops.kernels.elementwise.add import AddFwdKernel
from tileops.kernels.kernel_base import Kernel
from tileops.ops.op_base import Op

__all__ = ["AddFwdOp"]


class AddFwdOp(Op):
    """Element-wise ``y = input + alpha * other`` with broadcasting.

    Args:
        input, other: operand shapes (broadcast together).
        dtype: float16, bfloat16 or float32.
        alpha: Multiplier on ``other`` (default 1).
        kernel_map: Optional kernel dispatch override.
    """

    _op_name = "add"
    kernel_cls = AddFwdKernel
    _SUPPORTED_DTYPES = (torch.float16, torch.bfloat16, torch.float32)

    def __init__(self, *, input: tuple, other: tuple, dtype: torch.dtype, alpha=1,
                 kernel_map: Optional[Dict[str, Kernel]] = None):
        if dtype not in self._SUPPORTED_DTYPES:
            names = ", ".join(str(dt) for dt in self._SUPPORTED_DTYPES)
            raise ValueError(
                f"{type(self).__name__} does not support dtype {dtype}. Supported: [{names}]")
        self.input = tuple(input)
        self.other = tuple(other)
        self.input_shape = self.input
        self.other_shape = self.other
        self.dtype = dtype
        self.alpha = alpha
        self.output_dtype = dtype
        self.out_shape = tuple(torch.broadcast_shapes(self.input_shape, self.other_shape))
        self.N_total = prod(self.out_shape) if self.out_shape else 1
        self.dispatch_kernel(kernel_map)
        self.kernel = self.kernel_map[self._op_name](self.N_total, dtype, self.alpha)

    @property
    def default_kernel_map(self) -> Dict[str, Kernel]:
        return {self._op_name: self.kernel_cls}

    def forward(self, input: torch.Tensor, other: torch.Tensor) -> torch.Tensor:
        backend = get_device_backend()
        if not (backend.is_device_tensor(input) and backend.is_device_tensor(other)):
            raise ValueError(f"Inputs must be {backend.name} tensors")
        for name, t, expected in (("input", input, self.input_shape),
                                  ("other", other, self.other_shape)):
            if t.dtype != self.dtype:
                raise ValueError(f"Expected {name}.dtype {self.dtype}, got {t.dtype}")
            if tuple(t.shape) != expected:
                raise ValueError(f"Expected {name}.shape {expected}, got {tuple(t.shape)}")
        return self.kernel(input, other)

    def eval_roofline(self) -> tuple[int, int]:
        n_total = int(self.N_total)
        flops = (1 if self.alpha == 1 else 2) * n_total
        return flops, 3 * n_total * self.dtype.itemsize

