"""MishFwdOp: y = x * tanh(softplus(x)).

Reference: examples/TileOPs/tileops/ops/elementwise/mish.py:27-107
(``inplace`` flag; manifest flops ``4 * N``, bytes ``2 * N * elem_bytes``).
"""

from tileops.kernels.elementwise.mish import MishFwdKernel
from tileops.ops.elementwise._unary import InplaceActivationOp

__all__ = ["MishFwdOp"]


class MishFwdOp(InplaceActivationOp):
    """Element-wise Mish over ``N_total`` elements.

    Args:
        N_total: Total number of elements (flattened input).
        dtype: float16, bfloat16 or float32.
        inplace: Write the result into ``input`` and return ``input``.
        kernel_map: Optional kernel dispatch override.
    """

    _op_name = "mish"
    kernel_cls = MishFwdKernel
    FLOPS_PER_ELEM = 4
