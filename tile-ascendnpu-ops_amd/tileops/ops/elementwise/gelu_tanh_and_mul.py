"""GeluTanhAndMulFwdOp: y = gelu_tanh(x[:, :N]) * x[:, N:].

Reference: examples/TileOPs/tileops/ops/elementwise/gelu_tanh_and_mul.py:43-126
(manifest flops ``10 * M * N``, bytes ``3 * M * N * elem_bytes``).
"""

from tileops.kernels.elementwise.gelu_tanh_and_mul import GeluTanhAndMulFwdKernel
from tileops.ops.elementwise._gated import GatedActivationOp

__all__ = ["GeluTanhAndMulFwdOp"]


class GeluTanhAndMulFwdOp(GatedActivationOp):
    """Fused gated tanh-GELU (same arguments as GeluAndMulFwdOp)."""

    _op_name = "gelu_tanh_and_mul"
    kernel_cls = GeluTanhAndMulFwdKernel
    FLOPS_PER_OUTPUT = 10
