from tileops.kernels.elementwise.isfinite.isfinite import IsfiniteFwdKernel

__all__ = ["IsfiniteFwdKernel"]
