from tileops.kernels.elementwise.sub.sub import SubFwdKernel

__all__ = ["SubFwdKernel"]
