"""HardswishFwdKernel: y = x * clamp(x + 3, 0, 6) / 6 on gfx950.

Reference class: examples/TileOPs/tileops/kernels/elementwise/hardswish/hardswish.py:82-156.
Device code: unary_vec_kernel<T, TILEOPS_HARDSWISH> in csrc/elementwise.hip.
"""

from tileops.kernels.elementwise._streaming import HARDSWISH, UnaryFwdKernel

__all__ = ["HardswishFwdKernel"]


class HardswishFwdKernel(UnaryFwdKernel):
    """Hardswish forward kernel over ``N_total`` flattened elements.

    Args:
        N_total: Total number of elements (flattened input).
        dtype: float16, bfloat16 or float32.
        config: Optional config override.
    """

    _unary_op = HARDSWISH
