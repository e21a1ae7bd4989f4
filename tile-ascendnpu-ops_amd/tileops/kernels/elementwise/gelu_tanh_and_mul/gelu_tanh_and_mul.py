"""GeluTanhAndMulFwdKernel: y = gelu_tanh(x[:, :N]) * x[:, N:] on gfx950.

Reference class:
examples/TileOPs/tileops/kernels/elementwise/gelu_tanh_and_mul/gelu_tanh_and_mul.py:74-.
"""

from tileops.kernels.elementwise._streaming import GatedGeluFwdKernel

__all__ = ["GeluTanhAndMulFwdKernel"]


class GeluTanhAndMulFwdKernel(GatedGeluFwdKernel):
    """Fused gated tanh-GELU; ``x`` is ``(M, 2 * N)``, output ``(M, N)``."""

    _approx = 1
