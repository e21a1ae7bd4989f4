from tileops.kernels.elementwise.isinf.isinf import IsinfFwdKernel

__all__ = ["IsinfFwdKernel"]
