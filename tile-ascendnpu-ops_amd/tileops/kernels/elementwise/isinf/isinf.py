"""IsinfFwdKernel: bool infinity predicate on gfx950 (exact IEEE bit test).

Reference class: examples/TileOPs/tileops/kernels/elementwise/isinf/isinf.py.
The kernel writes one 0/1 byte per element straight into torch.bool storage.
"""

from tileops.kernels.elementwise._streaming import ISINF, PredicateFwdKernel

__all__ = ["IsinfFwdKernel"]


class IsinfFwdKernel(PredicateFwdKernel):
    """torch.isinf over ``N_total`` flattened float16 / bfloat16 / float32 elements."""

    _predicate = ISINF
