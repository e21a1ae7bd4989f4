"""AddFwdKernel / SubFwdKernel: y = a +- alpha * b with broadcasting on gfx950.

Reference classes: examples/TileOPs/tileops/kernels/elementwise/add, sub
(``(N_total, dtype, alpha, config=None)``; torch.add / torch.sub with fp32
opmath).  The reference Ops materialised the broadcast with
``expand().contiguous()`` and ran a flat kernel; here the kernel reads each
operand through per-dimension strides (0 on a broadcast dimension), so no
copy is made.  Device code: add_vec_kernel / add_bcast_kernel in
csrc/elementwise.hip (subtraction passes -alpha, which is exact).
"""

import ctypes
from typing import Optional, Sequence

import torch

from tileops import _native
from tileops.kernels.kernel_base import Kernel

__all__ = ["AddFwdKernel", "SubFwdKernel", "broadcast_strides"]

_MAX_DIMS = 8


def broadcast_strides(t: torch.Tensor, out_shape: Sequence[int]) -> list:
    """Element strides of ``t`` over the dims of ``out_shape`` (right-aligned,
    as torch broadcasting aligns them), 0 where ``t`` is broadcast."""
    nd, td = len(out_shape), t.dim()
    strides = [0] * nd
    for k in range(td):
        o = nd - td + k
        strides[o] = 0 if (t.shape[k] == 1 and out_shape[o] != 1) else t.stride(k)
    return strides


class AddFwdKernel(Kernel):
    """y = a + alpha * b over the broadcast shape of the operands.

    Args:
        N_total: Elements of the broadcast output.
        dtype: float16, bfloat16 or float32.
        alpha: Multiplier on ``b``.
        config: Optional config override.
    """

    supported_archs: Optional[list] = None
    SUPPORTED_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
    profile_kernel_name = "add_"
    _sign = 1.0

    def __init__(self, N_total: int, dtype: torch.dtype, alpha=1, config: Optional[dict] = None):
        super().__init__()
        if dtype not in self.SUPPORTED_DTYPES:
            names = ", ".join(str(dt) for dt in self.SUPPORTED_DTYPES)
            raise ValueError(f"{type(self).__name__} only supports dtypes [{names}], got {dtype}")
        self.N_total = int(N_total)
        self.dtype = dtype
        self.alpha = alpha
        self.init_config(config)

    @property
    def default_config(self) -> dict:
        return {"vector_bytes": 16, "max_dims": _MAX_DIMS}

    def forward(self, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        _native.require_device(a, b)
        out_shape = tuple(torch.broadcast_shapes(a.shape, b.shape))
        if len(out_shape) > _MAX_DIMS:
            raise ValueError(f"{type(self).__name__} supports at most {_MAX_DIMS} dims")
        n = 1
        for d in out_shape:
            n *= d
        if n != self.N_total:
            raise ValueError(f"Expected {self.N_total} output elements, got {n}")
        y = torch.empty(out_shape, dtype=self.dtype, device=a.device)
        nd = len(out_shape)
        shape = (ctypes.c_int64 * max(nd, 1))(*out_shape)
        sa = (ctypes.c_int64 * max(nd, 1))(*broadcast_strides(a, out_shape))
        sb = (ctypes.c_int64 * max(nd, 1))(*broadcast_strides(b, out_shape))
        code = _native.lib().tileops_add_fwd(
            a.data_ptr(), b.data_ptr(), y.data_ptr(), nd, shape, sa, sb,
            float(self._sign * self.alpha), _native.dtype_code(self.dtype), _native.stream_of(a))
        _native.check(code, type(self).__name__)
        return y


class SubFwdKernel(AddFwdKernel):
    """y = a - alpha * b (``torch.sub``): the add kernel with -alpha."""

    _sign = -1.0

