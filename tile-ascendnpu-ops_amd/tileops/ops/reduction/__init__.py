from tileops.ops.reduction.argmax import ArgmaxFwdOp
from tileops.ops.reduction.softmax import LogSumExpFwdOp

__all__ = ["ArgmaxFwdOp", "LogSumExpFwdOp"]
