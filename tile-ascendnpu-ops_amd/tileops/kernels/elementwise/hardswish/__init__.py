from tileops.kernels.elementwise.hardswish.hardswish import HardswishFwdKernel

__all__ = ["HardswishFwdKernel"]
