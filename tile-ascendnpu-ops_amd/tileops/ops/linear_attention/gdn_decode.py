"""GatedDeltaNetDecodeFwdOp: single-token gated delta-rule (GDN) decode.

The decode step beside GatedDeltaNetPrefillFwdOp, on its state layout.  The
reference has no GDN decode op; the step is one token of
golden_gdn_sequential (examples/gdn_prefill/probe/gdn_prefill_probe.py:60-77)
and the interface follows GLADecodeOp
(tileops/ops/linear_attention/gla_decode.py:24-77).  Per (batch, head)::

    S' = exp(g) S + beta k (v - k^T exp(g) S)^T
    o  = scale * q^T S'

``forward(q, k, v, g, beta, state) -> (o, new_state)`` with q, k
``[B, H, K]``, v / o ``[B, H, V]`` (one dtype), g, beta ``[B, H]`` fp32 and
states ``[B, H, K, V]`` fp32, returned functionally.  A prefill's
``final_state`` is a valid ``state``, and token t of a ``[B, T, H, D]``
sequence is ``q[:, t]``.  Roofline: ``B H (7 K V + 2 K + 7 V)`` flops and
the state read and written once (``8 K V`` bytes per head) plus q, k, v, o,
g and beta.
"""

from typing import Dict, Optional

import torch

from tileops.kernels.kernel_base import Kernel
from tileops.kernels.linear_attention.gdn_decode import GDNDecodeKernel
from tileops.ops.op_base import Op

__all__ = ["GatedDeltaNetDecodeFwdOp"]


class GatedDeltaNetDecodeFwdOp(Op):
    """Single-step (decode) gated DeltaNet, layout BHD.

    Args:
        batch: Batch size.
        heads: Number of heads.
        dim_k: Key / query head dim (a multiple of 32, at most 256).
        dim_v: Value head dim (a multiple of 32, at most 4096).
        dtype: q / k / v / o dtype (float16, bfloat16 or float32).
        scale: Output scale (default ``dim_k ** -0.5``).
        kernel_map: Optional kernel override.
    """

    _op_name = "gdn_decode"

    def __init__(
        self,
        batch: int,
        heads: int,
        dim_k: int = 128,
        dim_v: int = 128,
        dtype: torch.dtype = torch.bfloat16,
        scale: Optional[float] = None,
        *,
        kernel_map: Optional[Dict[str, Kernel]] = None,
    ) -> None:
        self.batch = batch
        self.heads = heads
        self.dim_k = dim_k
        self.dim_v = dim_v
        self.dtype = dtype
        self.scale = dim_k**-0.5 if scale is None else scale
        self.dispatch_kernel(kernel_map)
        self.kernel: Kernel = self.kernel_map[self._op_name](
            batch, heads, dim_k, dim_v, dtype, self.scale
        )

    @property
    def default_kernel_map(self) -> Dict[str, Kernel]:
        return {self._op_name: GDNDecodeKernel}

    def forward(
        self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
        beta: torch.Tensor, state: torch.Tensor,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """Run one decode step; returns ``(o, new_state)``."""
        return self.kernel(q, k, v, g, beta, state)

    def eval_roofline(self) -> tuple[int, int]:
        K, V, BH = self.dim_k, self.dim_v, self.batch * self.heads
        elem = self.dtype.itemsize
        flops = BH * (7 * K * V + 2 * K + 7 * V)
        nbytes = BH * (8 * K * V + (2 * K + 2 * V) * elem + 8)
        return int(flops), int(nbytes)
