"""IsnanFwdOp: y = torch.isnan(x) as a bool tensor.

Reference: examples/TileOPs/tileops/ops/elementwise/isnan.py:36-115 (float16 /
bfloat16 / float32 only; manifest flops ``N``, bytes ``N * (elem_bytes + 1)``).
"""

from tileops.kernels.elementwise.isnan import IsnanFwdKernel
from tileops.ops.elementwise._unary import PredicateOp

__all__ = ["IsnanFwdOp"]


class IsnanFwdOp(PredicateOp):
    """Element-wise NaN predicate over ``N_total`` elements (bool output).

    Args:
        N_total: Total number of elements (flattened input).
        dtype: Input dtype (float16, bfloat16 or float32).
        kernel_map: Optional kernel dispatch override.
    """

    _op_name = "isnan"
    kernel_cls = IsnanFwdKernel
    FLOPS_PER_ELEM = 1
