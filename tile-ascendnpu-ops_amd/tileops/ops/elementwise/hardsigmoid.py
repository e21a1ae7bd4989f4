"""HardsigmoidFwdOp: y = clamp(x + 3, 0, 6) / 6.

Reference: examples/TileOPs/tileops/ops/elementwise/hardsigmoid.py:27-107
(manifest flops ``3 * N``, bytes ``2 * N * elem_bytes``).
"""

from tileops.kernels.elementwise.hardsigmoid import HardsigmoidFwdKernel
from tileops.ops.elementwise._unary import InplaceActivationOp

__all__ = ["HardsigmoidFwdOp"]


class HardsigmoidFwdOp(InplaceActivationOp):
    """Element-wise HardSigmoid over ``N_total`` elements (``inplace`` as Hardswish)."""

    _op_name = "hardsigmoid"
    kernel_cls = HardsigmoidFwdKernel
    FLOPS_PER_ELEM = 3
