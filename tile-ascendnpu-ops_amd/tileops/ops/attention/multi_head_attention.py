"""MultiHeadAttentionFwdOp: BSHD multi-head attention forward -> (output, lse).

Reference: examples/TileOPs/tileops/ops/attention/multi_head_attention.py:34-120.
MHA is the ``heads_kv == heads`` case of the GQA prefill kernel, built at
construction with ``sm_scale = dim ** -0.5`` and ``softcap = 0``; the roofline
is ``4 * B * H * S^2 * D`` flops (halved when causal) and
``2 * (q_elems + kv_elems) * elem_bytes`` bytes.
"""

from typing import Dict, Optional

import torch

from tileops.kernels.attention.multi_head_attention import GQAPrefillFwdKernel
from tileops.kernels.kernel_base import Kernel
from tileops.ops.op_base import Op

__all__ = ["MultiHeadAttentionFwdOp"]


class MultiHeadAttentionFwdOp(Op):
    """Multi-head attention forward.  Layout: BSHD.

    Args:
        batch: Batch size.
        heads: Number of heads.
        seq_len: Query and key/value length.
        dim: Head dimension (64 or 128).
        is_causal: Apply the causal mask.
        dtype: float16 or bfloat16.
        kernel_map: Optional kernel override.
    """

    def __init__(
        self,
        batch: int,
        heads: int,
        seq_len: int,
        dim: int,
        is_causal: bool = True,
        dtype: torch.dtype = torch.float16,
        kernel_map: Optional[Dict[str, Kernel]] = None,
    ) -> None:
        self.batch = batch
        self.heads = heads
        self.seq_len = seq_len
        self.dim = dim
        self.is_causal = is_causal
        self.dtype = dtype
        self.dispatch_kernel(kernel_map)
        self.kernel: Kernel = self.kernel_map["gqa_prefill_fwd_kernel"](
            batch, heads, heads, seq_len, seq_len, dim, is_causal, dtype,
            sm_scale=dim**-0.5, softcap=0.0,
        )

    @property
    def default_kernel_map(self) -> Dict[str, Kernel]:
        return {"gqa_prefill_fwd_kernel": GQAPrefillFwdKernel}

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
        """BSHD q / k / v -> ``(output, lse)``."""
        return self.kernel(q, k, v)

    def eval_roofline(self) -> tuple[int, int]:
        elem = self.dtype.itemsize
        flops = 4 * self.batch * self.heads * self.seq_len * self.seq_len * self.dim
        if self.is_causal:
            flops //= 2
        q_elems = self.batch * self.seq_len * self.heads * self.dim
        return int(flops), int(2 * (q_elems + q_elems) * elem)
