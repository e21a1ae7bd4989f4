"""GLADecodeKernel: single-token gated linear attention decode on gfx950.

Reference: examples/TileOPs/tileops/kernels/linear_attention/gla_decode/
gla_decode.py:22-66 (constructor ``(B, H, DK, DV, dtype, scale, k_tile,
config)``, a non-positive ``scale`` meaning ``DK ** -0.5``, ``forward(q, k, v,
gk, state) -> (o, new_state)``) and the golden golden_gla_decode
(gla_decode_kernel/_gla_decode_kernel.py:211-218).  Layout BHD: q, k, gk
``[B, H, DK]``, v ``[B, H, DV]``, state ``[B, H, DK, DV]``, all one dtype.
Device code: gla_decode_rows_kernel (16-byte row slices, the common shapes)
or gla_decode_kernel in csrc/gla.hip.  ``k_tile`` is accepted for interface
parity; the HIP kernels stream whole rows and need no tiling.
"""

from typing import Optional, Tuple

import torch

from tileops import _native
from tileops.kernels.kernel_base import Kernel

__all__ = ["GLADecodeKernel"]


@torch.library.custom_op("tileops::gla_decode_fwd", mutates_args=())
def _gla_decode_fwd(
    B: int, H: int, DK: int, DV: int, scale: float,
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, gk: torch.Tensor, state: torch.Tensor,
) -> Tuple[torch.Tensor, torch.Tensor]:
    o = torch.empty_like(v)
    new_state = torch.empty_like(state)
    code = _native.lib().tileops_gla_decode_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), gk.data_ptr(), state.data_ptr(),
        o.data_ptr(), new_state.data_ptr(), B, H, DK, DV, float(scale),
        _native.dtype_code(q.dtype), _native.stream_of(q),
    )
    _native.check(code, "tileops_gla_decode_fwd")
    return o, new_state


@_gla_decode_fwd.register_fake
def _(B, H, DK, DV, scale, q, k, v, gk, state):
    return torch.empty_like(v), torch.empty_like(state)


class GLADecodeKernel(Kernel):
    """Single-step (decode) gated linear attention, layout BHD.

    Args:
        B, H, DK, DV: batch / heads / key dim / value dim.
        dtype: float16, bfloat16 or float32.
        scale: readout scale; non-positive means ``DK ** -0.5``.
        k_tile: accepted for interface parity; the kernel streams the whole
            state in one pass, so it selects nothing.
        config: Optional config override.
    """

    SUPPORTED_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
    profile_kernel_name = r"gla(?:::|\d+)gla_decode_(?:rows_)?kernel"

    def __init__(
        self,
        B: int,
        H: int,
        DK: int,
        DV: int,
        dtype: torch.dtype = torch.bfloat16,
        scale: float = -1.0,
        k_tile: Optional[int] = None,
        config: Optional[dict] = None,
    ) -> None:
        super().__init__()
        if dtype not in self.SUPPORTED_DTYPES:
            supported = ", ".join(str(dt) for dt in self.SUPPORTED_DTYPES)
            raise ValueError(
                f"{self.__class__.__name__} only supports dtypes [{supported}], got {dtype}"
            )
        if min(B, H, DK, DV) <= 0:
            raise ValueError("B > 0 and H > 0 and DK > 0 and DV > 0")
        self.B = B
        self.H = H
        self.DK = DK
        self.DV = DV
        self.dtype = dtype
        self.scale = float(scale) if scale is not None and scale > 0 else DK**-0.5
        self.k_tile = DK if k_tile is None else k_tile
        self.init_config(config)

    @property
    def default_config(self) -> dict:
        # 256-thread workgroups, one or more per (batch, head)
        return {"threads": 256}

    def forward(
        self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, gk: torch.Tensor,
        state: torch.Tensor,
    ) -> Tuple[torch.Tensor, torch.Tensor]:
        _native.require_device(q, k, v, gk, state)
        B, H, DK, DV = self.B, self.H, self.DK, self.DV
        for name, t, shape in (("q", q, (B, H, DK)), ("k", k, (B, H, DK)), ("v", v, (B, H, DV)),
                               ("gk", gk, (B, H, DK)), ("state", state, (B, H, DK, DV))):
            if tuple(t.shape) != shape:
                raise ValueError(f"Expected {name}.shape {shape}, got {tuple(t.shape)}")
            if t.dtype != self.dtype:
                raise ValueError(f"Expected {name}.dtype {self.dtype}, got {t.dtype}")
        q, k, v, gk, state = (t.contiguous() for t in (q, k, v, gk, state))
        return _gla_decode_fwd(B, H, DK, DV, self.scale, q, k, v, gk, state)
