from tileops.kernels.linear_attention.gla_decode.gla_decode import GLADecodeKernel

__all__ = ["GLADecodeKernel"]
