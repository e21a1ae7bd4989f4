from tileops.kernels.elementwise.hardsigmoid.hardsigmoid import HardsigmoidFwdKernel

__all__ = ["HardsigmoidFwdKernel"]
