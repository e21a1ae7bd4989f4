from tileops.kernels.elementwise.gelu_and_mul.gelu_and_mul import GeluAndMulFwdKernel

__all__ = ["GeluAndMulFwdKernel"]
