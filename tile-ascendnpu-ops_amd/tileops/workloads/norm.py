"""Workloads of the norm family (reference: examples/TileOPs/tileops/workloads/norm.py:36-59)."""

from typing import Optional

import torch

from tileops.device import get_device_backend
from tileops.workloads.workload_base import WorkloadBase


class FusedAddLayerNormWorkload(WorkloadBase):
    """``x`` / ``residual`` of shape ``(m, n)`` and affine ``weight`` / ``bias`` ``(n,)``.

    By default every operand is ``randn`` in ``dtype`` (the reference draw).
    ``param_dtype=torch.float32`` gives the mixed-precision layout with
    ``weight ~ N(1, 0.1^2)`` and ``bias ~ N(0, 0.1^2)`` in fp32.
    """

    def __init__(
        self,
        m: int,
        n: int,
        dtype: torch.dtype,
        eps: float = 1e-5,
        param_dtype: Optional[torch.dtype] = None,
    ):
        self.m = m
        self.n = n
        self.dtype = dtype
        self.eps = eps
        self.param_dtype = param_dtype

    def gen_inputs(self) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
        device = get_device_backend().name
        x = torch.randn(self.m, self.n, dtype=self.dtype, device=device)
        residual = torch.randn(self.m, self.n, dtype=self.dtype, device=device)
        if self.param_dtype is None:
            weight = torch.randn(self.n, dtype=self.dtype, device=device)
            bias = torch.randn(self.n, dtype=self.dtype, device=device)
        else:
            weight = (1.0 + 0.1 * torch.randn(self.n, device=device)).to(self.param_dtype)
            bias = (0.1 * torch.randn(self.n, device=device)).to(self.param_dtype)
        return x, residual, weight, bias
