"""ClampMinFwdOp: y = clamp_min(x, min) = max(x, min), NaN-propagating.

Reference: examples/TileOPs/tileops/ops/elementwise/clamp_min.py:35-117 --
``torch.clamp_min(input, min)`` is ``torch.clamp(input, min, max=None)``, so
the Op reuses the scalar-bound clamp kernel with no upper bound (manifest
flops ``1 * N``, bytes ``2 * N * elem_bytes``; ``min=None`` is rejected with
"ClampMinFwdOp requires min").
"""

from typing import Dict, Optional

import torch

from tileops.kernels.elementwise.clamp_scalar import ClampScalarFwdKernel
from tileops.kernels.kernel_base import Kernel
from tileops.ops.elementwise._unary import FlatElementwiseOp

__all__ = ["ClampMinFwdOp"]


class ClampMinFwdOp(FlatElementwiseOp):
    """Element-wise lower-bound clamp over ``N_total`` elements.

    Args:
        N_total: Total number of elements.
        dtype: float16, bfloat16 or float32.
        min: Lower bound (required).
        kernel_map: Optional kernel dispatch override.
    """

    _op_name = "clamp_min"
    kernel_cls = ClampScalarFwdKernel
    FLOPS_PER_ELEM = 1

    def __init__(
        self,
        N_total: int,
        dtype: torch.dtype,
        min: Optional[float] = None,
        *,
        kernel_map: Optional[Dict[str, Kernel]] = None,
    ):
        if min is None:
            raise ValueError("ClampMinFwdOp requires min")
        self.N_total = N_total
        self.dtype = dtype
        self.min = min
        self.max = None
        self.output_dtype = dtype
        self.dispatch_kernel(kernel_map)
        self.kernel = self.kernel_map[self._op_name](N_total, dtype, min, None)
