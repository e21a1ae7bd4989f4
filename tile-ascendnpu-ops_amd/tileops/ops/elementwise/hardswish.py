"""HardswishFwdOp: y = x * clamp(x + 3, 0, 6) / 6.

Reference: examples/TileOPs/tileops/ops/elementwise/hardswish.py:27-107
(manifest flops ``4 * N``, bytes ``2 * N * elem_bytes``).
"""

from tileops.kernels.elementwise.hardswish import HardswishFwdKernel
from tileops.ops.elementwise._unary import InplaceActivationOp

__all__ = ["HardswishFwdOp"]


class HardswishFwdOp(InplaceActivationOp):
    """Element-wise HardSwish over ``N_total`` elements.

    Args:
        N_total: Total number of elements (flattened input).
        dtype: float16, bfloat16 or float32.
        inplace: Write the result into ``input`` and return ``input``.
        kernel_map: Optional kernel dispatch override.
    """

    _op_name = "hardswish"
    kernel_cls = HardswishFwdKernel
    FLOPS_PER_ELEM = 4
