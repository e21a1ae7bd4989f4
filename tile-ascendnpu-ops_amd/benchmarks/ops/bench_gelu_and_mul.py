"""Benchmarks of GeluAndMulFwdOp over its manifest workloads (reference bench file:
examples/TileOPs/benchmarks/ops/bench_gelu_and_mul.py).  The op has one (M, 2N)
input, so the (M, N) workload rows are expanded here."""

import pytest
import torch

from tileops.benchmark.benchmark_base import BenchmarkReport, ManifestBenchmark
from tileops.manifest import load_workloads
from tileops.ops.elementwise.gelu_and_mul import GeluAndMulFwdOp
from tileops.workloads.elementwise import GeluAndMulWorkload

_OP = "GeluAndMulFwdOp"


def _params(workloads: list[dict]) -> list:
    return [pytest.param(w["M"], w["N"], getattr(torch, d), id=f"{w.get('label', 'manifest')}-{d}")
            for w in workloads for d in w["dtypes"]]


@pytest.mark.parametrize("M, N, dtype", _params(load_workloads(_OP)))
def test_gelu_and_mul_bench(M: int, N: int, dtype: torch.dtype) -> None:
    test = GeluAndMulWorkload(M, N, dtype)
    inputs = test.gen_inputs()
    op = GeluAndMulFwdOp(M=M, N=N, dtype=dtype)
    bm = ManifestBenchmark(_OP, op, test)
    result = bm.profile(op, *inputs)
    BenchmarkReport.record(op, locals(), result, tag="tileops")


if __name__ == "__main__":
    pytest.main([__file__, "-vvs"])
