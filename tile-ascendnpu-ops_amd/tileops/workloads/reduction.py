"""Workloads of the reduction family (reference: examples/TileOPs/tileops/workloads/reduction.py:6-11)."""

from tileops.workloads.workload_base import RandnWorkload


class LogSumExpWorkload(RandnWorkload):
    """Input of LogSumExpFwdOp (shape + dtype, randn)."""


class ArgmaxWorkload(RandnWorkload):
    """Input of ArgmaxFwdOp (shape + dtype, randn)."""
