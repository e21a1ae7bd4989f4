"""Benchmarks of SubFwdOp over its manifest workloads (reference bench file:
examples/TileOPs/benchmarks/ops/bench_sub.py)."""

import pytest
import torch

from tileops.benchmark.benchmark_base import BenchmarkReport, ManifestBenchmark
from tileops.manifest import load_workloads
from tileops.ops.elementwise.sub import SubFwdOp
from tileops.workloads.elementwise import BinaryWorkload

_OP = "SubFwdOp"


def _params(workloads: list[dict]) -> list:
    return [pytest.param(tuple(w["input_shape"]), tuple(w["other_shape"]), getattr(torch, d),
                         id=f"{w.get('label', 'manifest')}-{d}")
            for w in workloads for d in w["dtypes"]]


@pytest.mark.parametrize("input_shape, other_shape, dtype", _params(load_workloads(_OP)))
def test_sub_bench(input_shape: tuple, other_shape: tuple, dtype: torch.dtype) -> None:
    test = BinaryWorkload(input_shape, other_shape, dtype)
    inputs = test.gen_inputs()
    op = SubFwdOp(input=input_shape, other=other_shape, dtype=dtype)
    bm = ManifestBenchmark(_OP, op, test)
    result = bm.profile(op, *inputs)
    BenchmarkReport.record(op, locals(), result, tag="tileops")


if __name__ == "__main__":
    pytest.main([__file__, "-vvs"])
