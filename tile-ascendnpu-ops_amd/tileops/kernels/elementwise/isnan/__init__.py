from tileops.kernels.elementwise.isnan.isnan import IsnanFwdKernel

__all__ = ["IsnanFwdKernel"]
