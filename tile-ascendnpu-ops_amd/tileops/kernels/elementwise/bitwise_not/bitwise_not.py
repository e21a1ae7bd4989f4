"""BitwiseNotFwdKernel: y = ~x (torch.bitwise_not) on gfx950.

Reference class: examples/TileOPs/tileops/kernels/elementwise/bitwise_not/
bitwise_not.py (``BitwiseNotFwdKernel(N_total, dtype)`` over bool / integer
dtypes).  Device code: bitnot_vec_kernel / bitnot_byte_kernel in
csrc/elementwise.hip, a byte stream: integer bytes complemented, bool bytes
XOR 1.
"""

from typing import Optional

import torch

from tileops import _native
from tileops.kernels.kernel_base import Kernel

__all__ = ["BitwiseNotFwdKernel", "BITWISE_DTYPES"]

BITWISE_DTYPES = (torch.bool, torch.uint8, torch.int8, torch.int16, torch.int32, torch.int64)


class BitwiseNotFwdKernel(Kernel):
    """Bitwise NOT over ``N_total`` flattened bool / integer elements.

    Args:
        N_total: Total number of elements.
        dtype: bool, uint8, int8, int16, int32 or int64.
        config: Optional config override.
    """

    SUPPORTED_DTYPES = BITWISE_DTYPES
    profile_kernel_name = r"tileops(?:::|\d+)bitnot_(vec|byte)_kernel"

    def __init__(self, N_total: int, dtype: torch.dtype, config: Optional[dict] = None):
        super().__init__()
        if dtype not in self.SUPPORTED_DTYPES:
            names = ", ".join(str(dt) for dt in self.SUPPORTED_DTYPES)
            raise ValueError(f"{type(self).__name__} only supports dtypes [{names}], got {dtype}")
        self.N_total = int(N_total)
        self.dtype = dtype
        self.output_dtype = dtype
        self.init_config(config)

    @property
    def default_config(self) -> dict:
        # bitnot_vec_kernel: 256-thread workgroups, one 16-byte pack per thread
        return {"threads": 256, "vector_bytes": 16}

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        _native.require_device(x)
        self.check_tensor("x", x, dtype=self.dtype, numel=self.N_total)
        x = x.contiguous()
        y = torch.empty_like(x)
        code = _native.lib().tileops_bitwise_not_fwd(
            x.data_ptr(), y.data_ptr(), self.N_total * x.element_size(),
            1 if self.dtype == torch.bool else 0, _native.stream_of(x))
        _native.check(code, type(self).__name__)
        return y
