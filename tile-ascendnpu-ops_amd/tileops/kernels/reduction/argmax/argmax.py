"""ArgreduceKernel: row-wise argmax / argmin returning int64 on gfx950.

Reference class: examples/TileOPs/tileops/kernels/reduction/argmax/argmax.py:89-219.
Semantics are torch.argmax / torch.argmin: first occurrence among equal
values, NaN counts as the extreme value.  The launch is wrapped in the
``tileops::argreduce_fwd`` custom op (reference: ``npub::argreduce_fwd``).
Device code: row_reduce_kernel<T, 1|2, ...> in csrc/reduction.hip.
"""

from typing import Optional

import torch

from tileops import _native
from tileops.kernels.kernel_base import Kernel

__all__ = ["ArgreduceKernel"]

_ARGREDUCE_KINDS = {"argmax", "argmin"}


@torch.library.custom_op("tileops::argreduce_fwd", mutates_args=())
def _argreduce_fwd(M: int, N: int, op_kind: str, x: torch.Tensor) -> torch.Tensor:
    y = torch.empty((M,), dtype=torch.int64, device=x.device)
    code = _native.lib().tileops_argreduce_fwd(
        x.data_ptr(),
        y.data_ptr(),
        M,
        N,
        _native.dtype_code(x.dtype),
        1 if op_kind == "argmin" else 0,
        _native.stream_of(x),
    )
    _native.check(code, "tileops_argreduce_fwd")
    return y


@_argreduce_fwd.register_fake
def _(M: int, N: int, op_kind: str, x: torch.Tensor) -> torch.Tensor:
    return torch.empty((M,), dtype=torch.int64, device=x.device)


class ArgreduceKernel(Kernel):
    """Argmax / argmin forward kernel; output is always int64.

    Args:
        M: Number of rows.
        N: Reduction length.
        op_kind: ``"argmax"`` or ``"argmin"``.
        dtype: float32, float16 or bfloat16.
        config: Optional config override.
        device_index: Accepted for API compatibility.
    """

    profile_kernel_name = r"tileops(?:::|\d+)row_reduce_kernel"

    def __init__(
        self,
        M: int,
        N: int,
        op_kind: str,
        dtype: torch.dtype,
        config: Optional[dict] = None,
        device_index: Optional[int] = None,
    ):
        super().__init__()
        if op_kind not in _ARGREDUCE_KINDS:
            raise ValueError(
                f"Unsupported op_kind '{op_kind}'. Expected one of {sorted(_ARGREDUCE_KINDS)}."
            )
        self.M = M
        self.N = N
        self.op_kind = op_kind
        self.dtype = dtype
        self.device_index = device_index
        self.init_config(config)

    @property
    def default_config(self) -> dict:
        if self.N == 0:
            raise ValueError(
                "Reduction dimension is empty (N=0). "
                "argmax/argmin over an empty dimension is undefined."
            )
        # row_reduce_kernel: as LogSumExpKernel
        return {"wavefronts_per_row": 1 if self.M >= 3072 else 4, "packs_in_flight": 4}

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        _native.require_device(x)
        self.check_tensor("x", x, dtype=self.dtype, shape=(self.M, self.N))
        x = x.contiguous()
        return _argreduce_fwd(self.M, self.N, self.op_kind, x)
