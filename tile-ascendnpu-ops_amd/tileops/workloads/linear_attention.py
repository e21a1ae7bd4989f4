"""Workloads of the linear-attention family: GDN prefill inputs."""

import torch
import torch.nn.functional as F

from tileops.device import get_device_backend
from tileops.workloads.workload_base import WorkloadBase

__all__ = ["GdnPrefillWorkload"]


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
