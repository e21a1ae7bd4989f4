"""SubFwdKernel: y = a - alpha * b with broadcasting on gfx950.

Reference class: examples/TileOPs/tileops/kernels/elementwise/sub
(``(N_total, dtype, alpha, config=None)``; torch.sub with fp32 opmath).  It is
the add kernel with the multiplier negated, which is exact: torch.sub computes
a + (-alpha) b in the same single fma.
"""

from tileops.kernels.elementwise.add.add import AddFwdKernel

__all__ = ["SubFwdKernel"]


class SubFwdKernel(AddFwdKernel):
    """y = a - alpha * b (``torch.sub``)."""

    _sign = -1.0
