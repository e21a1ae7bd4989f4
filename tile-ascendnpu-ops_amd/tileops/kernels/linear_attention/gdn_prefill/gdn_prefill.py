"""GDNPrefillFwdKernel: chunked gated delta-rule prefill on gfx950.

The reference never delivered this kernel (MIGRATION_INDEX.md:28); the
recurrence follows golden_gdn_sequential
(examples/gdn_prefill/probe/gdn_prefill_probe.py:60-77) and the chunked WY
form of examples/gdn_prefill/DESIGN.md:6-17.  Layout is ``[B, T, H, D]``
(token-major, as ``chunk_gated_delta_rule`` takes it): q, k: ``[B, T, H, K]``
bf16, v: ``[B, T, H, V]`` bf16, g (log-decay) and beta: ``[B, T, H]`` fp32,
initial / final state ``[B, H, K, V]`` fp32.  The sequence runs in
segments (config ``segments``: 0 lets the library choose from the head
count and the device's compute units): one launch runs segment 0 exactly
and the state maps of the inner segments, a second composes each later
segment's start state and runs it exactly.  The workspace holds the maps
(64 KiB per map and head).  Device code: gdn_fused_kernel in csrc/gdn.hip.
"""

from typing import Optional, Tuple

import torch

from tileops import _native
from tileops.kernels.kernel_base import Kernel

__all__ = ["GDNPrefillFwdKernel"]


class GDNPrefillFwdKernel(Kernel):
    """Gated DeltaNet chunked prefill forward kernel.

    Args:
        batch, seq_len, heads: problem shape.
        dim_k, dim_v: key / value head dims (128 each).
        chunk_size: chunk length (64).
        dtype: q / k / v / o dtype (bfloat16).
        scale: output scale (default ``dim_k ** -0.5``).
        config: Optional config override.
    """

    SUPPORTED_DTYPES = (torch.bfloat16,)
    tunable_config = ("segments",)
    profile_kernel_name = r"gdn(?:::|\d+)gdn_(fused|compose|copy_state)_kernel"

    def __init__(
        self,
        batch: int,
        seq_len: int,
        heads: int,
        dim_k: int,
        dim_v: int,
        chunk_size: int = 64,
        dtype: torch.dtype = torch.bfloat16,
        scale: Optional[float] = None,
        config: Optional[dict] = None,
    ):
        super().__init__()
        if dtype not in self.SUPPORTED_DTYPES:
            supported = ", ".join(str(dt) for dt in self.SUPPORTED_DTYPES)
            raise ValueError(
                f"{self.__class__.__name__} only supports dtypes [{supported}], got {dtype}"
            )
        if dim_k != 128 or dim_v != 128 or chunk_size != 64:
            raise ValueError(
                f"{self.__class__.__name__} supports dim_k = dim_v = 128 and chunk_size = 64, "
                f"got {dim_k}, {dim_v}, {chunk_size}"
            )
        self.batch = batch
        self.seq_len = seq_len
        self.heads = heads
        self.dim_k = dim_k
        self.dim_v = dim_v
        self.chunk_size = chunk_size
        self.dtype = dtype
        self.scale = dim_k**-0.5 if scale is None else scale
        self.init_config(config)

    @property
    def default_config(self) -> dict:
        # sequence segments run in parallel (0: the library's choice)
        return {"chunk_size": self.chunk_size, "segments": 0}

    def workspace_bytes(self) -> int:
        return int(
            _native.lib().tileops_gdn_prefill_workspace_bytes_ex(
                self.batch, self.seq_len, self.heads, self.dim_k, self.dim_v, self.chunk_size,
                int(self.config.get("segments", 0)),
            )
        )

    def forward(
        self,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        g: torch.Tensor,
        beta: torch.Tensor,
        initial_state: Optional[torch.Tensor] = None,
        workspace: Optional[torch.Tensor] = None,
    ) -> Tuple[torch.Tensor, torch.Tensor]:
        _native.require_device(q, k, v, g, beta, initial_state)
        B, T, H = self.batch, self.seq_len, self.heads
        for name, t, shape, dt in (
            ("q", q, (B, T, H, self.dim_k), self.dtype),
            ("k", k, (B, T, H, self.dim_k), self.dtype),
            ("v", v, (B, T, H, self.dim_v), self.dtype),
            ("g", g, (B, T, H), torch.float32),
            ("beta", beta, (B, T, H), torch.float32),
        ):
            if tuple(t.shape) != shape:
                raise ValueError(f"Expected {name}.shape {shape}, got {tuple(t.shape)}")
            if t.dtype != dt:
                raise ValueError(f"Expected {name}.dtype {dt}, got {t.dtype}")
        if initial_state is not None:
            if tuple(initial_state.shape) != (B, H, self.dim_k, self.dim_v):
                raise ValueError(
                    f"Expected initial_state.shape {(B, H, self.dim_k, self.dim_v)}, "
                    f"got {tuple(initial_state.shape)}"
                )
            initial_state = initial_state.to(torch.float32).contiguous()
        q, k, v, g, beta = (t.contiguous() for t in (q, k, v, g, beta))
        o = torch.empty_like(v)
        final_state = torch.empty((B, H, self.dim_k, self.dim_v), dtype=torch.float32,
                                  device=q.device)
        need = self.workspace_bytes()
        if workspace is None or workspace.numel() < need:
            workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
        code = _native.lib().tileops_gdn_prefill_fwd_ex(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(),
            initial_state.data_ptr() if initial_state is not None else None,
            o.data_ptr(), final_state.data_ptr(),
            B, T, H, self.dim_k, self.dim_v, self.chunk_size, float(self.scale),
            _native.dtype_code(self.dtype), int(self.config.get("segments", 0)),
            workspace.data_ptr(), workspace.numel(), _native.stream_of(q),
        )
        _native.check(code, "tileops_gdn_prefill_fwd_ex")
        return o, final_state
