from tileops.kernels.reduction.argmax.argmax import ArgreduceKernel

__all__ = ["ArgreduceKernel"]
