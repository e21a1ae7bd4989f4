"""LogSumExpKernel: row-wise log-sum-exp over an (M, N) tensor on gfx950.

Reference class: examples/TileOPs/tileops/kernels/reduction/logsumexp/logsumexp.py:150-336.
y[i] = max_i + log(sum_j exp(x[i, j] - max_i)) in fp32, rounded to the input
dtype.  One wavefront folds each row with an online (max, scaled-sum) pair, so
any N works without host padding.  The launch is wrapped in the
``tileops::logsumexp_fwd`` custom op (with a fake impl) so ``torch.compile``
can trace through it, as the reference's ``npub::logsumexp_fwd`` did.
Device code: row_reduce_kernel<T, 0, ...> in csrc/reduction.hip.
"""

from typing import Optional

import torch

from tileops import _native
from tileops.kernels.kernel_base import Kernel

__all__ = ["LogSumExpKernel"]


@torch.library.custom_op("tileops::logsumexp_fwd", mutates_args=())
def _logsumexp_fwd(M: int, N: int, x: torch.Tensor) -> torch.Tensor:
    y = torch.empty((M,), dtype=x.dtype, device=x.device)
    code = _native.lib().tileops_logsumexp_fwd(
        x.data_ptr(), y.data_ptr(), M, N, _native.dtype_code(x.dtype), _native.stream_of(x)
    )
    _native.check(code, "tileops_logsumexp_fwd")
    return y


@_logsumexp_fwd.register_fake
def _(M: int, N: int, x: torch.Tensor) -> torch.Tensor:
    return torch.empty((M,), dtype=x.dtype, device=x.device)


class LogSumExpKernel(Kernel):
    """LogSumExp forward kernel.

    Args:
        M: Number of rows.
        N: Reduction length.
        op_kind: Must be ``"logsumexp"``.
        dtype: float32, float16 or bfloat16.
        config: Optional config override.
        device_index: Accepted for API compatibility (the kernel needs no
            per-device sizing).
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
        if op_kind != "logsumexp":
            raise ValueError(f"Unsupported op_kind '{op_kind}'. Expected 'logsumexp'.")
        self.M = M
        self.N = N
        self.op_kind = op_kind
        self.dtype = dtype
        self.device_index = device_index
        self.init_config(config)

    @property
    def default_config(self) -> dict:
        # row_reduce_kernel: 256-thread workgroups; one wavefront per row
        # (four rows per workgroup) from 3072 rows up, else the four
        # wavefronts of a workgroup share a row; 4 packs in flight per lane
        return {"wavefronts_per_row": 1 if self.M >= 3072 else 4, "packs_in_flight": 4}

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        _native.require_device(x)
        self.check_tensor("x", x, dtype=self.dtype, shape=(self.M, self.N))
        x = x.contiguous()
        return _logsumexp_fwd(self.M, self.N, x)
