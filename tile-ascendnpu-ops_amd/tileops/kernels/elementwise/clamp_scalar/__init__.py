from tileops.kernels.elementwise.clamp_scalar.clamp_scalar import ClampScalarFwdKernel

__all__ = ["ClampScalarFwdKernel"]
