from tileops.kernels.reduction.argmax import ArgreduceKernel
from tileops.kernels.reduction.logsumexp import LogSumExpKernel

__all__ = ["ArgreduceKernel", "LogSumExpKernel"]
