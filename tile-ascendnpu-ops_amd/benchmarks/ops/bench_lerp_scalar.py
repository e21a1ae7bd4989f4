"""Benchmarks of LerpFwdOp over its manifest workloads (reference bench file:
examples/TileOPs/benchmarks/ops/bench_lerp_scalar.py)."""

import pytest
import torch

from tileops.benchmark.benchmark_base import BenchmarkReport, ManifestBenchmark
from tileops.manifest import load_workloads
from tileops.ops.elementwise.lerp_scalar import LerpFwdOp
from tileops.workloads.elementwise import LerpScalarWorkload

_OP = "LerpFwdOp"


def _params(workloads: list[dict]) -> list:
    return [pytest.param(tuple(w["input_shape"]), tuple(w["end_shape"]), getattr(torch, d),
                         id=f"{w.get('label', 'manifest')}-{d}")
            for w in workloads for d in w["dtypes"]]


@pytest.mark.parametrize("input_shape, end_shape, dtype", _params(load_workloads(_OP)))
def test_lerp_scalar_bench(input_shape: tuple, end_shape: tuple, dtype: torch.dtype) -> None:
    test = LerpScalarWorkload(input_shape, end_shape, dtype)
    inputs = test.gen_inputs()
    op = LerpFwdOp(input=input_shape, end=end_shape, dtype=dtype, weight=0.3)
    bm = ManifestBenchmark(_OP, op, test)
    result = bm.profile(op, *inputs)
    BenchmarkReport.record(op, locals(), result, tag="tileops")


if __name__ == "__main__":
    pytest.main([__file__, "-vvs"])
