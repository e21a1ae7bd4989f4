from tileops.kernels.elementwise.mish.mish import MishFwdKernel

__all__ = ["MishFwdKernel"]
