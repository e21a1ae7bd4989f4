"""Workloads of the elementwise family.

Shapes and draws follow the reference
(examples/TileOPs/tileops/workloads/elementwise.py:11-323): shaped ``randn``
for the activations, a quarter each of NaN / +inf / -inf / finite for the
predicates, and one ``(M, 2 * N)`` tensor for the gated GELU ops.  Two extra
generators describe the MI355X benchmark inputs: a scaled normal draw
(``x ~ N(0, sigma^2)``) and special values scattered at seeded random positions.
"""

from math import prod

import torch

from tileops.device import get_device_backend
from tileops.workloads.workload_base import RandnWorkload, WorkloadBase


class ShapedRandnWorkload(RandnWorkload):
    """One ``randn`` tensor of any rank, with its element count ``n_total``."""

    def __init__(self, shape: tuple, dtype):
        super().__init__(tuple(shape), dtype)
        self.n_total = prod(self.shape)


class HardsigmoidWorkload(ShapedRandnWorkload):
    """Input of HardsigmoidFwdOp."""


class HardswishWorkload(ShapedRandnWorkload):
    """Input of HardswishFwdOp."""


class BinaryWorkload(WorkloadBase):
    """Operands of AddFwdOp / SubFwdOp: two randn tensors of their own shapes
    (broadcast together by the op)."""

    def __init__(self, input_shape: tuple, other_shape: tuple, dtype: torch.dtype):
        self.input_shape = tuple(input_shape)
        self.other_shape = tuple(other_shape)
        self.dtype = dtype
        self.n_total = prod(torch.broadcast_shapes(self.input_shape, self.other_shape))

    def gen_inputs(self):
        dev = get_device_backend().name
        return (torch.randn(self.input_shape, device=dev).to(self.dtype),
                torch.randn(self.other_shape, device=dev).to(self.dtype))


class AddWorkload(BinaryWorkload):
    """Operands of AddFwdOp (reference name: workloads/elementwise.py AddWorkload)."""


class SubWorkload(BinaryWorkload):
    """Operands of SubFwdOp (reference name: workloads/elementwise.py SubWorkload)."""


class LerpScalarWorkload(WorkloadBase):
    """Operands of LerpFwdOp: randn ``input`` and ``end`` of their own shapes
    (broadcast together by the op; the weight is an op parameter)."""

    def __init__(self, input_shape: tuple, end_shape: tuple, dtype: torch.dtype):
        self.input_shape = tuple(input_shape)
        self.end_shape = tuple(end_shape)
        self.shape = self.input_shape
        self.out_shape = tuple(torch.broadcast_shapes(self.input_shape, self.end_shape))
        self.n_total = prod(self.out_shape) if self.out_shape else 1
        self.dtype = dtype

    def gen_inputs(self):
        dev = get_device_backend().name
        return (torch.randn(self.input_shape, device=dev).to(self.dtype),
                torch.randn(self.end_shape, device=dev).to(self.dtype))


class LerpTensorManifestWorkload(WorkloadBase):
    """Operands of LerpTensorFwdOp at one manifest shape: randn ``input`` and
    ``end``, ``weight`` uniform on [0, 1) (interpolation weights)."""

    def __init__(self, shape: tuple, dtype: torch.dtype):
        self.shape = tuple(shape)
        self.input_shape = self.end_shape = self.weight_shape = self.shape
        self.n_total = prod(self.shape)
        self.dtype = dtype

    def gen_inputs(self):
        dev = get_device_backend().name
        return (torch.randn(self.shape, device=dev).to(self.dtype),
                torch.randn(self.shape, device=dev).to(self.dtype),
                torch.rand(self.shape, device=dev).to(self.dtype))


class BitwiseNotWorkload(WorkloadBase):
    """Input of BitwiseNotFwdOp: random bits of the dtype (bool: 0 / 1)."""

    def __init__(self, shape: tuple, dtype: torch.dtype):
        self.shape = tuple(shape)
        self.dtype = dtype
        self.n_total = prod(self.shape)

    def gen_inputs(self):
        dev = get_device_backend().name
        if self.dtype == torch.bool:
            return (torch.randint(0, 2, self.shape, device=dev).to(torch.bool),)
        nbytes = self.n_total * torch.empty(0, dtype=self.dtype).element_size()
        raw = torch.randint(0, 256, (nbytes,), device=dev, dtype=torch.uint8)
        return (raw.view(self.dtype).reshape(self.shape),)


class MishWorkload(ShapedRandnWorkload):
    """Input of MishFwdOp: randn of the workload shape."""


class ClampScalarWorkload(ShapedRandnWorkload):
    """Input of ClampScalarFwdOp (the bounds are op parameters)."""


class ScaledNormalWorkload(WorkloadBase):
    """``sigma * randn(shape)`` drawn in fp32 and rounded once to ``dtype``."""

    def __init__(self, shape: tuple, dtype: torch.dtype, sigma: float = 1.0):
        self.shape = tuple(shape)
        self.dtype = dtype
        self.sigma = sigma
        self.n_total = prod(self.shape)

    def gen_inputs(self) -> tuple[torch.Tensor]:
        device = get_device_backend().name
        x = torch.randn(self.shape, device=device, dtype=torch.float32)
        return ((x * self.sigma).to(self.dtype),)


class _QuarterSpecialWorkload(WorkloadBase):
    """Quarter NaN, quarter +inf, quarter -inf, rest ``randn`` (reference draw)."""

    def __init__(self, shape: tuple, dtype: torch.dtype):
        self.shape = tuple(shape)
        self.input_shape = self.shape
        self.n_total = prod(self.shape)
        self.dtype = dtype

    def gen_inputs(self) -> tuple[torch.Tensor]:
        device = get_device_backend().name
        x = torch.randn(self.shape, device=device, dtype=self.dtype)
        flat = x.view(-1)
        q = flat.numel() // 4
        flat[:q] = float("nan")
        flat[q : 2 * q] = float("inf")
        flat[2 * q : 3 * q] = float("-inf")
        return (x,)


class IsnanWorkload(_QuarterSpecialWorkload):
    """Input of IsnanFwdOp."""


class IsinfWorkload(_QuarterSpecialWorkload):
    """Input of IsinfFwdOp."""


class IsfiniteWorkload(_QuarterSpecialWorkload):
    """Input of IsfiniteFwdOp."""


class ScatteredSpecialWorkload(WorkloadBase):
    """``randn`` with ``inf_frac`` of the positions set to alternating +inf / -inf
    and ``nan_frac`` set to NaN, the positions drawn by a seeded permutation."""

    def __init__(
        self,
        shape: tuple,
        dtype: torch.dtype,
        inf_frac: float = 0.01,
        nan_frac: float = 0.01,
    ):
        self.shape = tuple(shape)
        self.dtype = dtype
        self.n_total = prod(self.shape)
        self.inf_frac = inf_frac
        self.nan_frac = nan_frac

    def gen_inputs(self) -> tuple[torch.Tensor]:
        device = get_device_backend().name
        x = torch.randn(self.shape, device=device, dtype=self.dtype)
        flat = x.view(-1)
        n = flat.numel()
        n_inf = int(n * self.inf_frac)
        n_nan = int(n * self.nan_frac)
        idx = torch.randperm(n, device=device)
        inf_idx = idx[:n_inf]
        signs = torch.where(
            torch.arange(n_inf, device=device) % 2 == 0,
            torch.tensor(float("inf"), device=device),
            torch.tensor(float("-inf"), device=device),
        ).to(self.dtype)
        flat[inf_idx] = signs
        flat[idx[n_inf : n_inf + n_nan]] = float("nan")
        return (x,)


class _GatedWorkload(WorkloadBase):
    """One ``(M, 2 * N)`` randn tensor: gate half then value half."""

    def __init__(self, M: int, N: int, dtype: torch.dtype):
        self.M = int(M)
        self.N = int(N)
        self.m = self.M
        self.n = self.N
        self.dtype = dtype
        self.x_shape = (self.M, 2 * self.N)
        self.shape = self.x_shape
        self.n_total = self.M * self.N

    def gen_inputs(self) -> tuple[torch.Tensor]:
        device = get_device_backend().name
        return (torch.randn(self.M, 2 * self.N, device=device, dtype=self.dtype),)


class GeluAndMulWorkload(_GatedWorkload):
    """Input of GeluAndMulFwdOp."""


class GeluTanhAndMulWorkload(_GatedWorkload):
    """Input of GeluTanhAndMulFwdOp."""
