from tileops.kernels.elementwise.lerp_tensor.lerp_tensor import LerpTensorFwdKernel

__all__ = ["LerpTensorFwdKernel"]
