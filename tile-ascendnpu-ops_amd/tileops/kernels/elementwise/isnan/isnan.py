"""IsnanFwdKernel: bool NaN predicate on gfx950 (exact IEEE bit test).

Reference class: examples/TileOPs/tileops/kernels/elementwise/isnan/isnan.py.
The kernel writes one 0/1 byte per element straight into torch.bool storage.
"""

from tileops.kernels.elementwise._streaming import ISNAN, PredicateFwdKernel

__all__ = ["IsnanFwdKernel"]


class IsnanFwdKernel(PredicateFwdKernel):
    """torch.isnan over ``N_total`` flattened float16 / bfloat16 / float32 elements."""

    _predicate = ISNAN
