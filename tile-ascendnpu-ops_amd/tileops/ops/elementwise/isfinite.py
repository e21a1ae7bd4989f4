"""IsfiniteFwdOp: y = torch.isfinite(x) as a bool tensor.

Reference: examples/TileOPs/tileops/ops/elementwise/isfinite.py:36-115 (float16 /
bfloat16 / float32 only; manifest flops ``N``, bytes ``N * (elem_bytes + 1)``).
"""

from tileops.kernels.elementwise.isfinite import IsfiniteFwdKernel
from tileops.ops.elementwise._unary import PredicateOp

__all__ = ["IsfiniteFwdOp"]


class IsfiniteFwdOp(PredicateOp):
    """Element-wise finiteness predicate over ``N_total`` elements (bool output).

    Args:
        N_total: Total number of elements (flattened input).
        dtype: Input dtype (float16, bfloat16 or float32).
        kernel_map: Optional kernel dispatch override.
    """

    _op_name = "isfinite"
    kernel_cls = IsfiniteFwdKernel
    FLOPS_PER_ELEM = 1
