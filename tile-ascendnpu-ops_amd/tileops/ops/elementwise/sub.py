"""SubFwdOp: y = input - alpha * other with PyTorch broadcasting.

Reference: examples/TileOPs/tileops/ops/elementwise/sub.py:37-
(constructor ``(*, input: shape, other: shape, dtype, alpha=1)``, float
dtypes, golden ``torch.sub(a.float(), b.float(), alpha=alpha).to(dtype)``;
roofline as AddFwdOp).  Shares AddFwdOp's flow with the subtraction kernel.
"""

from tileops.kernels.elementwise.sub import SubFwdKernel
from tileops.ops.elementwise.add import AddFwdOp

__all__ = ["SubFwdOp"]


class SubFwdOp(AddFwdOp):
    """Element-wise ``y = input - alpha * other`` with broadcasting.

    Args:
        input, other: operand shapes (broadcast together).
        dtype: float16, bfloat16 or float32.
        alpha: Multiplier on ``other`` (default 1).
        kernel_map: Optional kernel dispatch override.
    """

    _op_name = "sub"
    kernel_cls = SubFwdKernel
