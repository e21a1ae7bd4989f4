"""AddFwdKernel: y = a + alpha * b with broadcasting on gfx950.

Reference class: examples/TileOPs/tileops/kernels/elementwise/add
(``(N_total, dtype, alpha, config=None)``; torch.add with fp32 opmath).  The
reference Ops materialised the broadcast with ``expand().contiguous()`` and
ran a flat kernel; here the kernel reads each operand through per-dimension
strides (0 on a broadcast dimension), so no copy is made.  Device code:
bcast_vec_kernel / bcast_inner_kernel / bcast_any_kernel with BC_ADD in
csrc/elementwise.hip.
"""

import ctypes
from typing import Optional, Sequence

import torch

from tileops import _native
from tileops.kernels.kernel_base import Kernel

__all__ = ["AddFwdKernel", "BroadcastFwdKernel", "broadcast_strides", "MAX_DIMS"]

MAX_DIMS = 8


def broadcast_strides(t: torch.Tensor, out_shape: Sequence[int]) -> list:
    """Element strides of ``t`` over the dims of ``out_shape`` (right-aligned,
    as torch broadcasting aligns them), 0 where ``t`` is broadcast."""
    nd, td = len(out_shape), t.dim()
    strides = [0] * nd
    for k in range(td):
        o = nd - td + k
        strides[o] = 0 if (t.shape[k] == 1 and out_shape[o] != 1) else t.stride(k)
    return strides


class BroadcastFwdKernel(Kernel):
    """Shared flow of the broadcasting element-wise kernels: validate the
    operands, form the broadcast output shape and each operand's strides,
    and hand them to the C ABI as host arrays."""

    SUPPORTED_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
    profile_kernel_name = r"tileops(?:::|\d+)bcast_(vec|inner|any)_kernel"

    def _init_common(self, N_total: int, dtype: torch.dtype, config: Optional[dict]) -> None:
        if dtype not in self.SUPPORTED_DTYPES:
            names = ", ".join(str(dt) for dt in self.SUPPORTED_DTYPES)
            raise ValueError(f"{type(self).__name__} only supports dtypes [{names}], got {dtype}")
        self.N_total = int(N_total)
        self.dtype = dtype
        self.output_dtype = dtype
        self.init_config(config)

    @property
    def default_config(self) -> dict:
        # bcast_vec_kernel / bcast_inner_kernel: 256-thread workgroups, one
        # 16-byte pack per thread; operands of up to 8 broadcast dimensions
        return {"threads": 256, "vector_bytes": 16, "max_dims": MAX_DIMS}

    def _operands(self, names: Sequence[str], tensors: Sequence[torch.Tensor]):
        """``(out_shape, y, ndim, shape_arr, [stride_arr, ...])`` for the operands."""
        _native.require_device(*tensors)
        for name, t in zip(names, tensors):
            self.check_tensor(name, t, dtype=self.dtype)
        out_shape = tuple(torch.broadcast_shapes(*(t.shape for t in tensors)))
        if len(out_shape) > MAX_DIMS:
            raise ValueError(f"{type(self).__name__} supports at most {MAX_DIMS} dims")
        n = 1
        for d in out_shape:
            n *= d
        if n != self.N_total:
            raise ValueError(f"{type(self).__name__}: expected {self.N_total} output elements, "
                             f"got {n}")
        y = torch.empty(out_shape, dtype=self.dtype, device=tensors[0].device)
        nd = len(out_shape)
        arr = ctypes.c_int64 * max(nd, 1)
        strides = [arr(*broadcast_strides(t, out_shape)) for t in tensors]
        return out_shape, y, nd, arr(*out_shape), strides


class AddFwdKernel(BroadcastFwdKernel):
    """y = a + alpha * b over the broadcast shape of the operands.

    Args:
        N_total: Elements of the broadcast output.
        dtype: float16, bfloat16 or float32.
        alpha: Multiplier on ``b``.
        config: Optional config override.
    """

    _sign = 1.0

    def __init__(self, N_total: int, dtype: torch.dtype, alpha=1, config: Optional[dict] = None):
        super().__init__()
        self.alpha = alpha
        self._init_common(N_total, dtype, config)

    def forward(self, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        _shape, y, nd, shape, (sa, sb) = self._operands(("a", "b"), (a, b))
        code = _native.lib().tileops_add_fwd(
            a.data_ptr(), b.data_ptr(), y.data_ptr(), nd, shape, sa, sb,
            float(self._sign * self.alpha), _native.dtype_code(self.dtype), _native.stream_of(a))
        _native.check(code, type(self).__name__)
        return y
