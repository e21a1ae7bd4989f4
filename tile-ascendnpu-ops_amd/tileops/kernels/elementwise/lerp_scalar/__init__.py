from tileops.kernels.elementwise.lerp_scalar.lerp_scalar import LerpScalarFwdKernel

__all__ = ["LerpScalarFwdKernel"]
