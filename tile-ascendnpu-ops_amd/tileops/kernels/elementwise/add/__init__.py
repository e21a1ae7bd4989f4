from tileops.kernels.elementwise.add.add import AddFwdKernel

__all__ = ["AddFwdKernel"]
