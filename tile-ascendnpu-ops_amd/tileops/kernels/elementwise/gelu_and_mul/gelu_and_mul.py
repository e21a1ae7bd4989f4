"""GeluAndMulFwdKernel: y = gelu_erf(x[:, :N]) * x[:, N:] on gfx950.

Reference class: examples/TileOPs/tileops/kernels/elementwise/gelu_and_mul/gelu_and_mul.py:71-147.
One pass over x: each lane reads 16-byte packs of the gate and value halves.
"""

from tileops.kernels.elementwise._streaming import GatedGeluFwdKernel

__all__ = ["GeluAndMulFwdKernel"]


class GeluAndMulFwdKernel(GatedGeluFwdKernel):
    """Fused gated exact-GELU; ``x`` is ``(M, 2 * N)``, output ``(M, N)``."""

    _approx = 0
