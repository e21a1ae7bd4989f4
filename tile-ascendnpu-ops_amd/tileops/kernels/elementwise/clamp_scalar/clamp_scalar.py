"""ClampScalarFwdKernel: y = clamp(x, min, max) with scalar bounds on gfx950.

Reference class: examples/TileOPs/tileops/kernels/elementwise/clamp_scalar/clamp_scalar.py:82-190.
A bound that is ``None`` is not applied; at least one must be given.  The
bounds are applied in fp32 (the reference compares ``x.float()`` against
Python scalars), NaN inputs propagate and a NaN bound gives NaN everywhere.
"""

from typing import Optional

import torch

from tileops.kernels.elementwise._streaming import (
    CLAMP,
    CLAMP_HAS_MAX,
    CLAMP_HAS_MIN,
    UnaryFwdKernel,
)

__all__ = ["ClampScalarFwdKernel"]


class ClampScalarFwdKernel(UnaryFwdKernel):
    """Scalar-bound clamp over ``N_total`` flattened elements.

    Args:
        N_total: Total number of elements.
        dtype: float16, bfloat16 or float32.
        min_val: Lower bound or None.
        max_val: Upper bound or None (at least one bound is required).
        config: Optional config override.
    """

    _unary_op = CLAMP

    def __init__(
        self,
        N_total: int,
        dtype: torch.dtype,
        min_val: Optional[float] = None,
        max_val: Optional[float] = None,
        config: Optional[dict] = None,
    ):
        if min_val is None and max_val is None:
            raise ValueError("ClampScalarFwdKernel requires present(min) or present(max)")
        self.min_val = min_val
        self.max_val = max_val
        super().__init__(N_total, dtype, config)

    def _bounds(self) -> tuple[float, float, int]:
        flags = 0
        lo = hi = 0.0
        if self.min_val is not None:
            flags |= CLAMP_HAS_MIN
            lo = float(self.min_val)
        if self.max_val is not None:
            flags |= CLAMP_HAS_MAX
            hi = float(self.max_val)
        return lo, hi, flags
