"""GatedDeltaNetPrefillFwdOp: chunked gated delta-rule (GDN) prefill.

Delivery name and contract from the reference's migration plan
(MIGRATION_INDEX.md:28, 30; TileOPs迁移任务书.md:248-252): the operator of
``fla.ops.gated_delta_rule.chunk_gated_delta_rule``.  Per (batch, head)::

    S_t = exp(g_t) S_{t-1} + beta_t k_t (v_t - k_t^T exp(g_t) S_{t-1})^T
    o_t = scale * q_t^T S_t

``forward(q, k, v, g, beta, initial_state=None) -> (o, final_state)`` with
q, k ``[B, T, H, K]``, v / o ``[B, T, H, V]`` (bf16), g, beta ``[B, T, H]``
(fp32) and states ``[B, H, K, V]`` (fp32).  The roofline counts the chunked
WY algorithm, per chunk and head ``6 C^2 K + 4 C^2 V + 6 C K V + C^3 / 3``
flops, and the bytes of q, k, v, o, g, beta and the final state.
"""

from typing import Dict, Optional

import torch

from tileops.device import get_device_backend
from tileops.kernels.kernel_base import Kernel
from tileops.kernels.linear_attention.gdn_prefill import GDNPrefillFwdKernel
from tileops.ops.op_base import Op

__all__ = ["GatedDeltaNetPrefillFwdOp"]


class GatedDeltaNetPrefillFwdOp(Op):
    """Gated DeltaNet prefill forward.

    Args:
        batch: Batch size.
        seq_len: Tokens per sequence.
        heads: Number of heads.
        dim_k: Key / query head dim (128).
        dim_v: Value head dim (128).
        chunk_size: Chunk length of the WY form (64).
        dtype: q / k / v / o dtype (bfloat16).
        scale: Output scale (default ``dim_k ** -0.5``).
        kernel_map: Optional kernel override.
    """

    _op_name = "gdn_prefill"

    def __init__(
        self,
        batch: int,
        seq_len: int,
        heads: int,
        dim_k: int = 128,
        dim_v: int = 128,
        chunk_size: int = 64,
        dtype: torch.dtype = torch.bfloat16,
        scale: Optional[float] = None,
        *,
        kernel_map: Optional[Dict[str, Kernel]] = None,
    ):
        self.batch = batch
        self.seq_len = seq_len
        self.heads = heads
        self.dim_k = dim_k
        self.dim_v = dim_v
        self.chunk_size = chunk_size
        self.dtype = dtype
        self.scale = dim_k**-0.5 if scale is None else scale
        self.dispatch_kernel(kernel_map)
        self.kernel = self.kernel_map[self._op_name](
            batch, seq_len, heads, dim_k, dim_v, chunk_size, dtype, self.scale
        )
        self._workspace: Optional[torch.Tensor] = None

    @property
    def default_kernel_map(self) -> Dict[str, Kernel]:
        return {self._op_name: GDNPrefillFwdKernel}

    def forward(
        self,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        g: torch.Tensor,
        beta: torch.Tensor,
        initial_state: Optional[torch.Tensor] = None,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        backend = get_device_backend()
        for name, t in (("q", q), ("k", k), ("v", v), ("g", g), ("beta", beta)):
            if not backend.is_device_tensor(t):
                raise ValueError(f"{name} must be a {backend.name} tensor")
        need = self.kernel.workspace_bytes()
        if self._workspace is None or self._workspace.numel() < need:
            # kept across calls: the per-chunk workspace is reused
            self._workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
        return self.kernel(q, k, v, g, beta, initial_state, workspace=self._workspace)

    def eval_roofline(self) -> tuple[int, int]:
        C, K, V = self.chunk_size, self.dim_k, self.dim_v
        n_chunks = -(-self.seq_len // C) * self.batch * self.heads
        flops = (6 * C * C * K + 4 * C * C * V + 6 * C * K * V + C**3 // 3) * n_chunks
        tokens = self.batch * self.seq_len * self.heads
        elem = self.dtype.itemsize
        nbytes = (
            tokens * (2 * K + 2 * V) * elem  # q, k, v, o
            + tokens * 2 * 4  # g, beta
            + self.batch * self.heads * K * V * 4  # final state
        )
        return int(flops), int(nbytes)
