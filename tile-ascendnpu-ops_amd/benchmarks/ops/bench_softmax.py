"""Benchmarks of LogSumExpFwdOp over its manifest workloads (reference bench
file: examples/TileOPs/benchmarks/ops/bench_softmax.py, LogSumExp subset)."""

import pytest
import torch

from tileops.benchmark.benchmark_base import BenchmarkReport, ManifestBenchmark, workloads_to_params
from tileops.ops.reduction.softmax import LogSumExpFwdOp
from tileops.workloads.reduction import LogSumExpWorkload

_OP = "LogSumExpFwdOp"


@pytest.mark.parametrize("shape, dtype, op_params", workloads_to_params(_OP, include_extra=True))
def test_logsumexp_bench(shape: tuple, dtype: torch.dtype, op_params: dict) -> None:
    test = LogSumExpWorkload(shape, dtype)
    inputs = test.gen_inputs()
    op = LogSumExpFwdOp(dtype=dtype, **op_params)
    bm = ManifestBenchmark(_OP, op, test)
    result = bm.profile(op, *inputs)
    BenchmarkReport.record(op, locals(), result, tag="tileops")


if __name__ == "__main__":
    pytest.main([__file__, "-vvs"])
