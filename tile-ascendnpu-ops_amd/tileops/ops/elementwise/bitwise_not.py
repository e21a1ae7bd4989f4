"""BitwiseNotFwdOp: y = ~x for bool / integer inputs (torch.bitwise_not).

Reference: examples/TileOPs/tileops/ops/elementwise/bitwise_not.py:33-120
(admitted dtypes bool | uint8 | int8 | int16 | int32 | int64, the rejection
message "BitwiseNotFwdOp does not support dtype ...", manifest flops
``1 * N``, bytes ``2 * N * elem_bytes``).
"""

from typing import Dict, Optional

import torch

from tileops.kernels.elementwise.bitwise_not import BITWISE_DTYPES, BitwiseNotFwdKernel
from tileops.kernels.kernel_base import Kernel
from tileops.ops.elementwise._unary import FlatElementwiseOp

__all__ = ["BitwiseNotFwdOp"]


class BitwiseNotFwdOp(FlatElementwiseOp):
    """Element-wise bitwise NOT over ``N_total`` elements.

    Args:
        N_total: Total number of elements.
        dtype: bool, uint8, int8, int16, int32 or int64.
        kernel_map: Optional kernel dispatch override.
    """

    _op_name = "bitwise_not"
    kernel_cls = BitwiseNotFwdKernel
    FLOPS_PER_ELEM = 1
    _SUPPORTED_DTYPES = BITWISE_DTYPES

    def __init__(
        self,
        N_total: int,
        dtype: torch.dtype,
        *,
        kernel_map: Optional[Dict[str, Kernel]] = None,
    ):
        if dtype not in self._SUPPORTED_DTYPES:
            names = ", ".join(str(dt).replace("torch.", "") for dt in self._SUPPORTED_DTYPES)
            raise ValueError(f"BitwiseNotFwdOp does not support dtype {dtype}. Supported: [{names}]")
        self.N_total = N_total
        self.dtype = dtype
        self.output_dtype = dtype
        self.dispatch_kernel(kernel_map)
        self.kernel = self.kernel_map[self._op_name](N_total, dtype)
