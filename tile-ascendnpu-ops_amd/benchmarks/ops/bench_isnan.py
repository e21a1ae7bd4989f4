"""Benchmarks of IsnanFwdOp over its manifest workloads (reference bench file:
examples/TileOPs/benchmarks/ops/bench_isnan.py)."""

import pytest
import torch

from tileops.benchmark.benchmark_base import BenchmarkReport, ManifestBenchmark, workloads_to_params
from tileops.ops.elementwise.isnan import IsnanFwdOp
from tileops.workloads.elementwise import IsnanWorkload

_OP = "IsnanFwdOp"


@pytest.mark.parametrize("shape, dtype, op_params", workloads_to_params(_OP, include_extra=True))
def test_isnan_bench(shape: tuple, dtype: torch.dtype, op_params: dict) -> None:
    test = IsnanWorkload(shape, dtype)
    inputs = test.gen_inputs()
    op = IsnanFwdOp(N_total=test.n_total, dtype=dtype, **op_params)
    bm = ManifestBenchmark(_OP, op, test)
    result = bm.profile(op, *inputs)
    BenchmarkReport.record(op, locals(), result, tag="tileops")


if __name__ == "__main__":
    pytest.main([__file__, "-vvs"])
