"""Benchmarks of BitwiseNotFwdOp over its manifest workloads (reference bench file:
examples/TileOPs/benchmarks/ops/bench_bitwise_not.py)."""

import pytest
import torch

from tileops.benchmark.benchmark_base import BenchmarkReport, ManifestBenchmark, workloads_to_params
from tileops.ops.elementwise.bitwise_not import BitwiseNotFwdOp
from tileops.workloads.elementwise import BitwiseNotWorkload

_OP = "BitwiseNotFwdOp"


@pytest.mark.parametrize("shape, dtype, op_params", workloads_to_params(_OP, include_extra=True))
def test_bitwise_not_bench(shape: tuple, dtype: torch.dtype, op_params: dict) -> None:
    test = BitwiseNotWorkload(shape, dtype)
    inputs = test.gen_inputs()
    op = BitwiseNotFwdOp(N_total=test.n_total, dtype=dtype, **op_params)
    bm = ManifestBenchmark(_OP, op, test)
    result = bm.profile(op, *inputs)
    BenchmarkReport.record(op, locals(), result, tag="tileops")


if __name__ == "__main__":
    pytest.main([__file__, "-vvs"])
