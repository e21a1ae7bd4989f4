"""GDNDecodeKernel: single-token gated delta-rule (gated DeltaNet) decode on gfx950.

The reference has no GDN decode kernel; the step is one token of
golden_gdn_sequential (examples/gdn_prefill/probe/gdn_prefill_probe.py:60-77),
on the state layout of the GDN prefill (``[B, H, K, V]`` fp32), and the
interface follows GLADecodeKernel
(tileops/kernels/linear_attention/gla_decode/gla_decode.py:22-66) with
GDN's per-head gate and write strength: q, k ``[B, H, K]``, v ``[B, H, V]``
of one dtype, g (log-decay) and beta ``[B, H]`` fp32, state ``[B, H, K, V]``
fp32; ``forward(q, k, v, g, beta, state) -> (o, new_state)``.  Device code:
gdn_decode_kernel in csrc/gdn_decode.hip (one pass over the state).
"""

from typing import Optional, Tuple

import torch

from tileops import _native
from tileops.kernels.kernel_base import Kernel

__all__ = ["GDNDecodeKernel"]


@torch.library.custom_op("tileops::gdn_decode_fwd", mutates_args=())
def _gdn_decode_fwd(
    B: int, H: int, DK: int, DV: int, scale: float,
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor, beta: torch.Tensor,
    state: torch.Tensor,
) -> Tuple[torch.Tensor, torch.Tensor]:
    if state.data_ptr() % 16:  # the kernel moves the state in 16-byte packs
        state = state.clone()
    o = torch.empty_like(v)
    new_state = torch.empty_like(state)
    code = _native.lib().tileops_gdn_decode_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(),
        state.data_ptr(), o.data_ptr(), new_state.data_ptr(), B, H, DK, DV, float(scale),
        _native.dtype_code(q.dtype), _native.stream_of(q),
    )
    _native.check(code, "tileops_gdn_decode_fwd")
    return o, new_state


@_gdn_decode_fwd.register_fake
def _(B, H, DK, DV, scale, q, k, v, g, beta, state):
    return torch.empty_like(v), torch.empty_like(state)


class GDNDecodeKernel(Kernel):
    """Single-step (decode) gated DeltaNet, layout BHD.

    Args:
        batch, heads: problem shape.
        dim_k: key / query head dim (a multiple of 32, at most 256).
        dim_v: value head dim (a multiple of 32, at most 4096).
        dtype: q / k / v / o dtype (float16, bfloat16 or float32).
        scale: output scale (default ``dim_k ** -0.5``).
        config: Optional config override.
    """

    SUPPORTED_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
    profile_kernel_name = r"gdnd(?:::|\d+)gdn_decode_kernel"

    def __init__(
        self,
        batch: int,
        heads: int,
        dim_k: int = 128,
        dim_v: int = 128,
        dtype: torch.dtype = torch.bfloat16,
        scale: Optional[float] = None,
        config: Optional[dict] = None,
    ) -> None:
        super().__init__()
        if dtype not in self.SUPPORTED_DTYPES:
            supported = ", ".join(str(dt) for dt in self.SUPPORTED_DTYPES)
            raise ValueError(
                f"{self.__class__.__name__} only supports dtypes [{supported}], got {dtype}"
            )
        if min(batch, heads) <= 0:
            raise ValueError("batch > 0 and heads > 0")
        if dim_k <= 0 or dim_k % 32 or dim_k > 256 or dim_v <= 0 or dim_v % 32 or dim_v > 4096:
            raise ValueError(
                f"{self.__class__.__name__} needs dim_k a multiple of 32 up to 256 and dim_v a "
                f"multiple of 32 up to 4096, got {dim_k}, {dim_v}"
            )
        self.batch = batch
        self.heads = heads
        self.dim_k = dim_k
        self.dim_v = dim_v
        self.dtype = dtype
        self.scale = dim_k**-0.5 if scale is None else float(scale)
        self.init_config(config)

    @property
    def default_config(self) -> dict:
        # gdn_decode_kernel: 256-thread workgroups, each over 64 value columns
        # of a head where dim_v allows it (else 32)
        return {"threads": 256}

    def forward(
        self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
        beta: torch.Tensor, state: torch.Tensor,
    ) -> Tuple[torch.Tensor, torch.Tensor]:
        _native.require_device(q, k, v, g, beta, state)
        B, H, K, V = self.batch, self.heads, self.dim_k, self.dim_v
        for name, t, shape, dt in (
            ("q", q, (B, H, K), self.dtype),
            ("k", k, (B, H, K), self.dtype),
            ("v", v, (B, H, V), self.dtype),
            ("g", g, (B, H), torch.float32),
            ("beta", beta, (B, H), torch.float32),
            ("state", state, (B, H, K, V), torch.float32),
        ):
            if tuple(t.shape) != shape:
                raise ValueError(f"Expected {name}.shape {shape}, got {tuple(t.shape)}")
            if t.dtype != dt:
                raise ValueError(f"Expected {name}.dtype {dt}, got {t.dtype}")
        q, k, v, g, beta, state = (t.contiguous() for t in (q, k, v, g, beta, state))
        return _gdn_decode_fwd(B, H, K, V, self.scale, q, k, v, g, beta, state)
