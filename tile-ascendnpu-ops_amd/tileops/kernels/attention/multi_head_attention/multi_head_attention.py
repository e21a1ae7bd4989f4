"""GQAPrefillFwdKernel: flash-attention forward on gfx950 MFMA (BSHD layout).

Reference class:
examples/TileOPs/tileops/kernels/attention/multi_head_attention/multi_head_attention.py:132-.
Computes ``o = softmax(sm_scale * q k^T + causal mask) v`` and the per-row
log-sum-exp in the log2 domain (``logsumexp / ln 2``, shape
``[batch, heads, seq_len_q]``, float32), for ``heads % heads_kv == 0``.  The
causal mask is right-aligned (query i sees keys j <= i + Skv - Sq).  The
launch is wrapped in the ``tileops::gqa_prefill_fwd`` custom op (reference:
``npub::gqa_prefill_fwd_wrapped_kernel``).
Device code: mha_fwd_kernel in csrc/attention.hip.
"""

from typing import Optional, Tuple

import torch

from tileops import _native
from tileops.kernels.kernel_base import Kernel

__all__ = ["GQAPrefillFwdKernel"]


@torch.library.custom_op("tileops::gqa_prefill_fwd", mutates_args=())
def _gqa_prefill_fwd(
    batch: int,
    heads: int,
    heads_kv: int,
    seq_len_q: int,
    seq_len_kv: int,
    dim: int,
    is_causal: bool,
    sm_scale: float,
    softcap: float,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
) -> Tuple[torch.Tensor, torch.Tensor]:
    o = torch.empty_like(q)
    lse = torch.empty((batch, heads, seq_len_q), dtype=torch.float32, device=q.device)
    code = _native.lib().tileops_mha_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
        batch, seq_len_q, seq_len_kv, heads, heads_kv, dim,
        1 if is_causal else 0, float(sm_scale), float(softcap), _native.dtype_code(q.dtype),
        _native.stream_of(q),
    )
    _native.check(code, "tileops_mha_fwd")
    return o, lse


@_gqa_prefill_fwd.register_fake
def _(batch, heads, heads_kv, seq_len_q, seq_len_kv, dim, is_causal, sm_scale, softcap, q, k, v):
    return torch.empty_like(q), q.new_empty((batch, heads, seq_len_q), dtype=torch.float32)


class GQAPrefillFwdKernel(Kernel):
    """GQA / MHA prefill forward kernel (flash attention, BSHD).

    Args:
        batch, heads, heads_kv, seq_len_q, seq_len_kv, dim: problem shape
            (``dim`` 64, 96, 128, 192 or 256; ``heads % heads_kv == 0``).
        is_causal: Apply the right-aligned causal mask.
        dtype: float16 or bfloat16.
        sm_scale: Softmax scale (default ``dim ** -0.5``).
        softcap: Score soft-capping, ``softcap * tanh(scale q.k / softcap)`` before the
            mask and the softmax; ``0.0`` (default) turns it off.
        config: Optional config override.
    """

    SUPPORTED_DTYPES = (torch.float16, torch.bfloat16)
    profile_kernel_name = r"mha(?:::|\d+)mha_fwd_kernel"

    def __init__(
        self,
        batch: int,
        heads: int,
        heads_kv: int,
        seq_len_q: int,
        seq_len_kv: int,
        dim: int,
        is_causal: bool,
        dtype: torch.dtype,
        sm_scale: Optional[float] = None,
        softcap: float = 0.0,
        config: Optional[dict] = None,
    ) -> None:
        super().__init__()
        if heads % heads_kv != 0:
            raise ValueError("heads must be divisible by heads_kv")
        if is_causal and seq_len_q > seq_len_kv:
            raise ValueError("causal prefill requires seq_len_q <= seq_len_kv")
        if dtype not in self.SUPPORTED_DTYPES:
            supported = ", ".join(str(dt) for dt in self.SUPPORTED_DTYPES)
            raise ValueError(
                f"{self.__class__.__name__} only supports dtypes [{supported}], got {dtype}"
            )
        if dim not in (64, 96, 128, 192, 256):
            raise ValueError(
                f"{self.__class__.__name__} supports dim 64, 96, 128, 192 or 256, got {dim}"
            )
        if not (0.0 <= softcap < float("inf")):
            raise ValueError(f"{self.__class__.__name__}: softcap must be finite and >= 0 (got {softcap})")
        self.batch = batch
        self.heads = heads
        self.heads_kv = heads_kv
        self.seq_len_q = seq_len_q
        self.seq_len_kv = seq_len_kv
        self.dim = dim
        self.is_causal = is_causal
        self.dtype = dtype
        self.sm_scale = dim**-0.5 if sm_scale is None else sm_scale
        self.softcap = softcap
        self.init_config(config)

    @property
    def default_config(self) -> dict:
        # mha_fwd_kernel: 256 query rows per 512-thread workgroup (8
        # wavefronts x 32 rows); head dim 128: 128-key K / V tiles in two LDS
        # slots each; head dims 64 and 256: 64-key tiles in three slots
        if self.dim == 128:
            return {"block_m": 256, "block_n": 128, "num_stages": 2, "threads": 512}
        return {"block_m": 256, "block_n": 64, "num_stages": 3, "threads": 512}

    def forward(
        self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor
    ) -> Tuple[torch.Tensor, torch.Tensor]:
        _native.require_device(q, k, v)
        exp_q = (self.batch, self.seq_len_q, self.heads, self.dim)
        exp_kv = (self.batch, self.seq_len_kv, self.heads_kv, self.dim)
        if tuple(q.shape) != exp_q:
            raise ValueError(f"Expected q.shape {exp_q}, got {tuple(q.shape)}")
        for name, t in (("k", k), ("v", v)):
            if tuple(t.shape) != exp_kv:
                raise ValueError(f"Expected {name}.shape {exp_kv}, got {tuple(t.shape)}")
        for name, t in (("q", q), ("k", k), ("v", v)):
            if t.dtype != self.dtype:
                raise ValueError(f"Expected {name}.dtype {self.dtype}, got {t.dtype}")
        return _gqa_prefill_fwd(
            self.batch, self.heads, self.heads_kv, self.seq_len_q, self.seq_len_kv, self.dim,
            self.is_causal, self.sm_scale, self.softcap, q.contiguous(), k.contiguous(),
            v.contiguous(),
        )
