from tileops.kernels.elementwise.add.add import AddFwdKernel, SubFwdKernel

__all__ = ["AddFwdKernel", "SubFwdKernel"]
