from tileops.kernels.elementwise.bitwise_not.bitwise_not import BITWISE_DTYPES, BitwiseNotFwdKernel

__all__ = ["BITWISE_DTYPES", "BitwiseNotFwdKernel"]
