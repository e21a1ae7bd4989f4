"""ArgmaxFwdOp: torch.argmax along one dim (or the flattened tensor), int64 out.

Reference: examples/TileOPs/tileops/ops/reduction/argmax.py:26-82 (scalar dim
or None only; list/tuple dims raise; roofline ``M * N`` flops,
``M * N * elem_bytes + M * 8`` bytes).
"""

from typing import Dict, Optional

import torch

from tileops.kernels.kernel_base import Kernel
from tileops.kernels.reduction.argmax import ArgreduceKernel
from tileops.ops.reduction.reduce import _ReduceOpBase

__all__ = ["ArgmaxFwdOp"]


class ArgmaxFwdOp(_ReduceOpBase):
    """Argmax returning int64 indices (first occurrence; NaN is the maximum).

    Args:
        dtype: Input dtype.
        dim: Reduction dim, or None to index into the flattened tensor.
        keepdim: Keep the reduced dim(s) as size 1.
        kernel_map: Optional kernel override.
    """

    _op_kind = "argmax"
    _kernel_key = "argreduce"
    _kernel_cls = ArgreduceKernel

    def __init__(
        self,
        dtype: torch.dtype,
        dim: Optional[int] = None,
        keepdim: bool = False,
        *,
        kernel_map: Optional[Dict[str, Kernel]] = None,
    ):
        super().__init__(dtype=dtype, dim=dim, keepdim=keepdim, kernel_map=kernel_map)

    def _validate_dim(self) -> None:
        if self.dim is None or isinstance(self.dim, int):
            return
        raise ValueError(
            f"ArgmaxFwdOp only supports scalar dim (int) or None, "
            f"got {type(self.dim).__name__}: {self.dim!r}"
        )

    def _pad_value(self) -> float:
        return float("-inf")
