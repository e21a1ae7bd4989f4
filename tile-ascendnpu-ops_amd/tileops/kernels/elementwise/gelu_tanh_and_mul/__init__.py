from tileops.kernels.elementwise.gelu_tanh_and_mul.gelu_tanh_and_mul import GeluTanhAndMulFwdKernel

__all__ = ["GeluTanhAndMulFwdKernel"]
