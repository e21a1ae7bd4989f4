"""GeluAndMulFwdOp: y = gelu_erf(x[:, :N]) * x[:, N:].

Reference: examples/TileOPs/tileops/ops/elementwise/gelu_and_mul.py:42-125
(manifest flops ``6 * M * N``, bytes ``3 * M * N * elem_bytes``).
"""

from tileops.kernels.elementwise.gelu_and_mul import GeluAndMulFwdKernel
from tileops.ops.elementwise._gated import GatedActivationOp

__all__ = ["GeluAndMulFwdOp"]


class GeluAndMulFwdOp(GatedActivationOp):
    """Fused gated exact-GELU.

    Args:
        M: Rows of ``x`` and of the output.
        N: Output width; ``x`` has ``2 * N`` columns.
        dtype: float16, bfloat16 or float32.
        kernel_map: Optional kernel dispatch override.
    """

    _op_name = "gelu_and_mul"
    kernel_cls = GeluAndMulFwdKernel
    FLOPS_PER_OUTPUT = 6
