from tileops.kernels.linear_attention.gdn_decode.gdn_decode import GDNDecodeKernel

__all__ = ["GDNDecodeKernel"]
