"""IsinfFwdOp: y = torch.isinf(x) as a bool tensor.

Reference: examples/TileOPs/tileops/ops/elementwise/isinf.py:36-115 (float16 /
bfloat16 / float32 only; manifest flops ``N``, bytes ``N * (elem_bytes + 1)``).
"""

from tileops.kernels.elementwise.isinf import IsinfFwdKernel
from tileops.ops.elementwise._unary import PredicateOp

__all__ = ["IsinfFwdOp"]


class IsinfFwdOp(PredicateOp):
    """Element-wise infinity predicate over ``N_total`` elements (bool output).

    Args:
        N_total: Total number of elements (flattened input).
        dtype: Input dtype (float16, bfloat16 or float32).
        kernel_map: Optional kernel dispatch override.
    """

    _op_name = "isinf"
    kernel_cls = IsinfFwdKernel
    FLOPS_PER_ELEM = 1
