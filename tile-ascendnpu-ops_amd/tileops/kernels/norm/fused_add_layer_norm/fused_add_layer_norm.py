"""FusedAddLayerNormKernel: residual add + LayerNorm in one gfx950 kernel.

Reference class:
examples/TileOPs/tileops/kernels/norm/fused_add_layer_norm/fused_add_layer_norm.py:61-159.
Per row of N elements::

    residual_out = round_dtype(x + residual)
    y = round_dtype((residual_out - mean) * rsqrt(var + eps) * weight + bias)

with mean / biased variance of the rounded sum in fp32.  ``forward`` returns a
list ``[y, residual_out]`` shaped like ``x``.  ``weight`` / ``bias`` may be the
input dtype (the reference contract) or float32.
Device code (csrc/norm.hip): fused_add_ln_wave_kernel (up to 1024 16-byte
packs per row: one wavefront per row), fused_add_ln_block_kernel (1025 to
2048 packs: one 256-lane workgroup per row, the row in registers) and
fused_add_ln_generic_kernel (any other N or alignment).
"""

from typing import Optional

import torch

from tileops import _native
from tileops.kernels.kernel_base import Kernel

__all__ = ["FusedAddLayerNormKernel"]


class FusedAddLayerNormKernel(Kernel):
    """Fused add + LayerNorm forward kernel.

    Args:
        M: Number of rows (product of the leading dims of ``x``).
        N: Hidden dimension.
        eps: Variance epsilon.
        dtype: float32, float16 or bfloat16.
        config: Optional config override.
    """

    SUPPORTED_DTYPES = (torch.float32, torch.float16, torch.bfloat16)
    profile_kernel_name = r"tileops(?:::|\d+)fused_add_ln_(wave|block|generic)_kernel"

    def __init__(
        self,
        M: int,
        N: int,
        eps: float,
        dtype: torch.dtype,
        config: Optional[dict] = None,
    ):
        super().__init__()
        if dtype not in self.SUPPORTED_DTYPES:
            supported = ", ".join(str(dt) for dt in self.SUPPORTED_DTYPES)
            raise ValueError(
                f"{self.__class__.__name__} only supports dtypes [{supported}], got {dtype}"
            )
        self.M = M
        self.N = N
        self.eps = eps
        self.dtype = dtype
        self.init_config(config)

    @property
    def default_config(self) -> dict:
        # fused_add_ln_wave_kernel: one wavefront per row with the row held in
        # registers, four rows per 256-thread workgroup, weight / bias staged
        # in LDS as fp32 (longer rows: one 256-thread workgroup per row)
        return {"rows_per_wave": 1, "rows_per_workgroup": 4}

    def forward(
        self,
        x: torch.Tensor,
        residual: torch.Tensor,
        weight: torch.Tensor,
        bias: torch.Tensor,
    ) -> list[torch.Tensor]:
        _native.require_device(x, residual, weight, bias)
        self.check_tensor("x", x, dtype=self.dtype, numel=self.M * self.N)
        if x.dim() == 0 or x.shape[-1] != self.N:
            raise ValueError(f"{type(self).__name__}: expected x.shape[-1] == {self.N}, "
                             f"got {tuple(x.shape)}")
        self.check_tensor("residual", residual, dtype=self.dtype, shape=x.shape)
        self.check_tensor("weight", weight, numel=self.N)
        self.check_tensor("bias", bias, numel=self.N)
        original_shape = x.shape
        rows = x.contiguous().reshape(-1, self.N)
        res = residual.contiguous().reshape(-1, self.N)
        w = weight.contiguous().reshape(self.N)
        b = bias.contiguous().reshape(self.N)
        if w.dtype != b.dtype:
            raise ValueError(f"weight.dtype {w.dtype} != bias.dtype {b.dtype}")
        if w.dtype not in (self.dtype, torch.float32):
            raise ValueError(f"weight dtype must be {self.dtype} or torch.float32, got {w.dtype}")
        m = rows.shape[0]
        y = torch.empty_like(rows)
        r_out = torch.empty_like(rows)
        code = _native.lib().tileops_fused_add_layernorm_fwd(
            rows.data_ptr(),
            res.data_ptr(),
            w.data_ptr(),
            b.data_ptr(),
            y.data_ptr(),
            r_out.data_ptr(),
            m,
            self.N,
            float(self.eps),
            _native.dtype_code(self.dtype),
            _native.dtype_code(w.dtype),
            _native.stream_of(rows),
        )
        _native.check(code, "FusedAddLayerNormKernel")
        return [y.reshape(original_shape), r_out.reshape(original_shape)]
