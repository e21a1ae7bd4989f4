"""FusedAddLayerNormFwdOp: residual add + LayerNorm, returning (y, residual_out).

Reference: examples/TileOPs/tileops/ops/norm/fused_add_layer_norm.py:39-189.
Kept: constructor ``(M=None, N=None, dtype=None, eps=1e-5, kernel_map=None)``,
device / dtype / shape validation messages, ``contiguous().reshape(-1, N)``
flattening, the ``(M, N, dtype, device_index)`` kernel cache and the roofline
``8 * M * N`` flops, ``(4 * M * N + 2 * N) * elem_bytes`` bytes.

One extension: ``weight`` / ``bias`` may also be float32 when ``x`` is
float16 / bfloat16 (fp32 affine parameters are the common mixed-precision
layout); the roofline then counts their 4-byte elements.  Same-dtype
parameters behave exactly as in the reference.
"""

from typing import Dict, Optional

import torch

from tileops.device import get_device_backend
from tileops.kernels.kernel_base import Kernel
from tileops.kernels.norm import FusedAddLayerNormKernel
from tileops.ops.op_base import Op

__all__ = ["FusedAddLayerNormFwdOp"]


class FusedAddLayerNormFwdOp(Op):
    """Fused residual addition and LayerNorm.

    Args:
        M: Optional committed row count (product of the leading dims).
        N: Optional committed hidden dimension.
        dtype: float32, float16 or bfloat16 (inferred from ``x`` when None).
        eps: Variance epsilon.
        kernel_map: Optional kernel override dictionary.
    """

    _op_name = "fused_add_layer_norm"

    def __init__(
        self,
        M: Optional[int] = None,
        N: Optional[int] = None,
        dtype: Optional[torch.dtype] = None,
        eps: float = 1e-5,
        kernel_map: Optional[Dict[str, Kernel]] = None,
    ):
        self.M = M
        self.N = N
        self.dtype = dtype
        self._committed_M = M
        self._committed_N = N
        self._committed_dtype = dtype
        self.eps = eps
        self.dispatch_kernel(kernel_map)
        self._kernel_cache: Dict[tuple, Kernel] = {}
        self._last_roofline_mn: Optional[tuple[int, int]] = None
        self._last_param_bytes: Optional[int] = None

    @property
    def default_kernel_map(self) -> Dict[str, Kernel]:
        return {self._op_name: FusedAddLayerNormKernel}

    def eval_roofline(self) -> tuple[int, int]:
        if self._last_roofline_mn is None or self.dtype is None:
            raise RuntimeError(
                f"{type(self).__name__}.eval_roofline() requires a prior "
                "forward() call to bind input shape and dtype"
            )
        M, N = self._last_roofline_mn
        elem = self.dtype.itemsize
        param = self._last_param_bytes or elem
        return 8 * M * N, 4 * M * N * elem + 2 * N * param

    def _get_kernel(self, M: int, N: int, dtype: torch.dtype, device_index) -> Kernel:
        key = (M, N, dtype, device_index)
        if key not in self._kernel_cache:
            self._kernel_cache[key] = self.kernel_map[self._op_name](M, N, self.eps, dtype)
        return self._kernel_cache[key]

    def forward(
        self,
        x: torch.Tensor,
        residual: torch.Tensor,
        weight: torch.Tensor,
        bias: torch.Tensor,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        backend = get_device_backend()
        for name, t in (("x", x), ("residual", residual), ("weight", weight), ("bias", bias)):
            if not backend.is_device_tensor(t):
                raise ValueError(f"{name} must be a {backend.name} tensor")

        expected = self._committed_dtype
        if expected is not None and x.dtype != expected:
            raise ValueError(f"Expected x.dtype {expected}, got {x.dtype}")
        if expected is None:
            expected = x.dtype
        if residual.dtype != expected:
            raise ValueError(f"Expected residual.dtype {expected}, got {residual.dtype}")
        param_dtype = weight.dtype if weight.dtype == torch.float32 else expected
        for name, t in (("weight", weight), ("bias", bias)):
            if t.dtype != param_dtype:
                raise ValueError(f"Expected {name}.dtype {param_dtype}, got {t.dtype}")

        if residual.shape != x.shape:
            raise ValueError(f"Expected residual shape {x.shape}, got {residual.shape}")
        N = x.shape[-1]
        if tuple(weight.shape) != (N,):
            raise ValueError(f"Expected weight shape {(N,)}, got {tuple(weight.shape)}")
        if tuple(bias.shape) != (N,):
            raise ValueError(f"Expected bias shape {(N,)}, got {tuple(bias.shape)}")
        if self._committed_N is not None and self._committed_N != N:
            raise ValueError(f"Expected hidden dim {self._committed_N}, got {N}")

        orig_shape = x.shape
        x = x.contiguous().reshape(-1, N)
        residual = residual.contiguous().reshape(-1, N)
        weight = weight.contiguous().reshape(N)
        bias = bias.contiguous().reshape(N)
        M_actual = x.shape[0]
        if self._committed_M is not None and M_actual != self._committed_M:
            raise ValueError(
                f"Expected M={self._committed_M} (product of leading dims), got {M_actual}"
            )
        self.M = M_actual
        self.N = N
        self.dtype = expected

        kernel = self._get_kernel(M_actual, N, expected, x.device.index)
        y, residual_out = kernel(x, residual, weight, bias)
        self._last_roofline_mn = (M_actual, N)
        self._last_param_bytes = weight.dtype.itemsize
        return y.reshape(orig_shape), residual_out.reshape(orig_shape)
