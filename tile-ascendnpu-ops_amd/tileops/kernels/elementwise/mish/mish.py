"""MishFwdKernel: y = x * tanh(softplus(x)) on gfx950.

Reference class: examples/TileOPs/tileops/kernels/elementwise/mish/mish.py
(``MishFwdKernel(N_total, dtype)``; golden ``F.mish(x.float()).to(dtype)``,
tests/ops/test_mish.py:38-39).  Device code: unary_vec_kernel<T, TILEOPS_MISH>
in csrc/elementwise.hip, fp32 arithmetic rounded once.
"""

from tileops.kernels.elementwise._streaming import MISH, UnaryFwdKernel

__all__ = ["MishFwdKernel"]


class MishFwdKernel(UnaryFwdKernel):
    """Mish forward kernel over ``N_total`` flattened elements.

    Args:
        N_total: Total number of elements (flattened input).
        dtype: float16, bfloat16 or float32.
        config: Optional config override.
    """

    _unary_op = MISH
