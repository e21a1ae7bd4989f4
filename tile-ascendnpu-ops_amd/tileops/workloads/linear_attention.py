"""Workloads of the linear-attention family: GDN prefill and decode, GLA decode."""

import torch
import torch.nn.functional as F

from tileops.device import get_device_backend
from tileops.workloads.workload_base import WorkloadBase

__all__ = ["GdnDecodeWorkload", "GdnPrefillWorkload"]


class GdnPrefillWorkload(WorkloadBase):
    """q, k = L2-normalised randn per head, v = randn (``dtype``); g =
    logsigmoid(randn), beta = sigmoid(randn) (fp32); layout ``[B, T, H, D]``."""

    def __init__(self, batch: int, seq_len: int, heads: int, dim_k: int, dim_v: int,
                 dtype: torch.dtype = torch.bfloat16):
        self.batch = batch
        self.seq_len = seq_len
        self.heads = heads
        self.dim_k = dim_k
        self.dim_v = dim_v
        self.dtype = dtype

    def gen_inputs(self):
        device = get_device_backend().name
        B, T, H = self.batch, self.seq_len, self.heads
        q = F.normalize(torch.randn(B, T, H, self.dim_k, device=device), dim=-1).to(self.dtype)
        k = F.normalize(torch.randn(B, T, H, self.dim_k, device=device), dim=-1).to(self.dtype)
        v = torch.randn(B, T, H, self.dim_v, device=device).to(self.dtype)
        g = F.logsigmoid(torch.randn(B, T, H, device=device))
        beta = torch.sigmoid(torch.randn(B, T, H, device=device))
        return q, k, v, g, beta


class GdnDecodeWorkload(WorkloadBase):
    """One decode token per head, layout BHD: q, k = L2-normalised randn,
    v = randn (``dtype``); g = logsigmoid(randn), beta = sigmoid(randn)
    (fp32 ``[B, H]``); state = randn (fp32 ``[B, H, K, V]``)."""

    def __init__(self, batch: int, heads: int, dim_k: int, dim_v: int,
                 dtype: torch.dtype = torch.bfloat16):
        self.batch = batch
        self.heads = heads
        self.dim_k = dim_k
        self.dim_v = dim_v
        self.dtype = dtype

    def gen_inputs(self):
        device = get_device_backend().name
        B, H, K, V = self.batch, self.heads, self.dim_k, self.dim_v
        q = F.normalize(torch.randn(B, H, K, device=device), dim=-1).to(self.dtype)
        k = F.normalize(torch.randn(B, H, K, device=device), dim=-1).to(self.dtype)
        v = torch.randn(B, H, V, device=device).to(self.dtype)
        g = F.logsigmoid(torch.randn(B, H, device=device))
        beta = torch.sigmoid(torch.randn(B, H, device=device))
        state = torch.randn(B, H, K, V, device=device)
        return q, k, v, g, beta, state


class GLADecodeWorkload(WorkloadBase):
    """Single-token GLA decode inputs, layout BHD (tileops/workloads/
    linear_attention.py:19-47 of the reference): q, k, v ~ 0.5 N(0, 1),
    gk = -U[0, 1) (log-decay), state ~ N(0, 1), all of ``dtype``."""

    def __init__(self, B: int, H: int, DK: int, DV: int, dtype: torch.dtype,
                 scale: float = -1.0) -> None:
        self.B, self.H, self.DK, self.DV = B, H, DK, DV
        self.dtype = dtype
        self.scale = float(scale) if scale is not None and scale > 0 else DK**-0.5

    def gen_inputs(self):
        dev = get_device_backend().name
        B, H, DK, DV, dt = self.B, self.H, self.DK, self.DV, self.dtype
        q = (torch.randn(B, H, DK, device=dev, dtype=dt) * 0.5).contiguous()
        k = (torch.randn(B, H, DK, device=dev, dtype=dt) * 0.5).contiguous()
        v = (torch.randn(B, H, DV, device=dev, dtype=dt) * 0.5).contiguous()
        gk = (-torch.rand(B, H, DK, device=dev, dtype=dt)).contiguous()
        state = torch.randn(B, H, DK, DV, device=dev, dtype=dt).contiguous()
        return q, k, v, gk, state


def gla_decode_tolerance(dtype: torch.dtype) -> dict:
    """Tolerance of a GLA decode result against the fp32 golden (the
    reference's gla_decode_tolerance)."""
    if dtype == torch.float16:
        return {"atol": 2e-3, "rtol": 2e-3}
    if dtype == torch.bfloat16:
        return {"atol": 2e-2, "rtol": 2e-2}
    return {"atol": 1e-4, "rtol": 1e-4}
