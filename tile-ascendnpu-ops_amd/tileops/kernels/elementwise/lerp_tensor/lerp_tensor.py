"""LerpTensorFwdKernel: y = lerp(a, b, w) with a weight tensor on gfx950.

Reference class: examples/TileOPs/tileops/kernels/elementwise/lerp_tensor/lerp_tensor.py:90-180
(``(N_total, dtype, config=None)``, float dtypes; golden
``torch.lerp(a, b, w)``, tests/ops/test_lerp_tensor.py).  ``forward`` takes
the three operands flat (``N_total`` elements each) or broadcastable to
``N_total`` elements, read through strides without a materialised copy.
Device code: the broadcast kernels of csrc/elementwise.hip with
BC_LERP_TENSOR.
"""

from typing import Optional

import torch

from tileops import _native
from tileops.kernels.elementwise.add.add import BroadcastFwdKernel

__all__ = ["LerpTensorFwdKernel"]


class LerpTensorFwdKernel(BroadcastFwdKernel):
    """Tensor-weight lerp over ``N_total`` output elements.

    Args:
        N_total: Elements of the (broadcast) output.
        dtype: float16, bfloat16 or float32 (all three operands).
        config: Optional config override.
    """

    def __init__(self, N_total: int, dtype: torch.dtype, config: Optional[dict] = None):
        super().__init__()
        self._init_common(N_total, dtype, config)

    def forward(self, a: torch.Tensor, b: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        _shape, y, nd, shape, (sa, sb, sw) = self._operands(("a", "b", "w"), (a, b, w))
        code = _native.lib().tileops_lerp_fwd(
            a.data_ptr(), b.data_ptr(), w.data_ptr(), y.data_ptr(), nd, shape, sa, sb, sw,
            0.0, _native.dtype_code(self.dtype), _native.stream_of(a))
        _native.check(code, type(self).__name__)
        return y
