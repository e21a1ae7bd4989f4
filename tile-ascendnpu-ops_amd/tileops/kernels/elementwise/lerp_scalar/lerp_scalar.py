"""LerpScalarFwdKernel: y = lerp(a, b, weight) with a scalar weight on gfx950.

Reference class: examples/TileOPs/tileops/kernels/elementwise/lerp_scalar/lerp_scalar.py:83-160
(``(N_total, dtype, weight=0.5, config=None)``, float dtypes, weight fixed at
construction; golden ``torch.lerp(a, b, weight)``,
tests/ops/test_lerp_scalar.py:58-60).  ``forward`` takes the two operands
either flat (``N_total`` elements each, as the reference kernel did) or
broadcastable to ``N_total`` elements: broadcast operands are read through
strides, never expanded into a copy.  Device code: the broadcast kernels of
csrc/elementwise.hip with BC_LERP_SCALAR (torch's two-sided lerp, each side
one fp32 fma).
"""

from typing import Optional

import torch

from tileops import _native
from tileops.kernels.elementwise.add.add import BroadcastFwdKernel

__all__ = ["LerpScalarFwdKernel"]


class LerpScalarFwdKernel(BroadcastFwdKernel):
    """Scalar-weight lerp over ``N_total`` output elements.

    Args:
        N_total: Elements of the (broadcast) output.
        dtype: float16, bfloat16 or float32.
        weight: Interpolation weight (default 0.5).
        config: Optional config override.
    """

    def __init__(self, N_total: int, dtype: torch.dtype, weight: float = 0.5,
                 config: Optional[dict] = None):
        super().__init__()
        self.weight = weight
        self._init_common(N_total, dtype, config)

    def forward(self, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        _shape, y, nd, shape, (sa, sb) = self._operands(("a", "b"), (a, b))
        code = _native.lib().tileops_lerp_fwd(
            a.data_ptr(), b.data_ptr(), None, y.data_ptr(), nd, shape, sa, sb, None,
            float(self.weight), _native.dtype_code(self.dtype), _native.stream_of(a))
        _native.check(code, type(self).__name__)
        return y
