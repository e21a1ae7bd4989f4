from tileops.kernels.reduction.logsumexp.logsumexp import LogSumExpKernel

__all__ = ["LogSumExpKernel"]
