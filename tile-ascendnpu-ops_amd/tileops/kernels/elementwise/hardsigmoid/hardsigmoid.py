"""HardsigmoidFwdKernel: y = clamp(x + 3, 0, 6) / 6 on gfx950 (NaN propagates).

Reference class: examples/TileOPs/tileops/kernels/elementwise/hardsigmoid/hardsigmoid.py:78-.
Device code: unary_vec_kernel<T, TILEOPS_HARDSIGMOID> in csrc/elementwise.hip.
"""

from tileops.kernels.elementwise._streaming import HARDSIGMOID, UnaryFwdKernel

__all__ = ["HardsigmoidFwdKernel"]


class HardsigmoidFwdKernel(UnaryFwdKernel):
    """Hardsigmoid forward kernel over ``N_total`` flattened elements."""

    _unary_op = HARDSIGMOID
