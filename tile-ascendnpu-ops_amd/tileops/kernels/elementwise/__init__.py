from tileops.kernels.elementwise.add import AddFwdKernel
from tileops.kernels.elementwise.bitwise_not import BitwiseNotFwdKernel
from tileops.kernels.elementwise.clamp_scalar import ClampScalarFwdKernel
from tileops.kernels.elementwise.gelu_and_mul import GeluAndMulFwdKernel
from tileops.kernels.elementwise.gelu_tanh_and_mul import GeluTanhAndMulFwdKernel
from tileops.kernels.elementwise.hardsigmoid import HardsigmoidFwdKernel
from tileops.kernels.elementwise.hardswish import HardswishFwdKernel
from tileops.kernels.elementwise.isfinite import IsfiniteFwdKernel
from tileops.kernels.elementwise.isinf import IsinfFwdKernel
from tileops.kernels.elementwise.isnan import IsnanFwdKernel
from tileops.kernels.elementwise.lerp_scalar import LerpScalarFwdKernel
from tileops.kernels.elementwise.lerp_tensor import LerpTensorFwdKernel
from tileops.kernels.elementwise.mish import MishFwdKernel
from tileops.kernels.elementwise.sub import SubFwdKernel

__all__ = [
    "AddFwdKernel",
    "BitwiseNotFwdKernel",
    "SubFwdKernel",
    "ClampScalarFwdKernel",
    "GeluAndMulFwdKernel",
    "GeluTanhAndMulFwdKernel",
    "HardsigmoidFwdKernel",
    "HardswishFwdKernel",
    "IsfiniteFwdKernel",
    "IsinfFwdKernel",
    "IsnanFwdKernel",
    "LerpScalarFwdKernel",
    "LerpTensorFwdKernel",
    "MishFwdKernel",
]
