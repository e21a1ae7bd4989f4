"""IsfiniteFwdKernel: bool finiteness predicate on gfx950 (exact IEEE bit test).

Reference class: examples/TileOPs/tileops/kernels/elementwise/isfinite/isfinite.py.
The kernel writes one 0/1 byte per element straight into torch.bool storage.
"""

from tileops.kernels.elementwise._streaming import ISFINITE, PredicateFwdKernel

__all__ = ["IsfiniteFwdKernel"]


class IsfiniteFwdKernel(PredicateFwdKernel):
    """torch.isfinite over ``N_total`` flattened float16 / bfloat16 / float32 elements."""

    _predicate = ISFINITE
