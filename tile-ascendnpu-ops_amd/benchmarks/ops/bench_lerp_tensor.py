"""Benchmarks of LerpTensorFwdOp over its manifest workloads (reference bench
file: examples/TileOPs/benchmarks/ops/bench_lerp_tensor.py)."""

import pytest
import torch

from tileops.benchmark.benchmark_base import BenchmarkReport, ManifestBenchmark
from tileops.manifest import load_workloads
from tileops.ops.elementwise.lerp_tensor import LerpTensorFwdOp
from tileops.workloads.elementwise import LerpTensorManifestWorkload

_OP = "LerpTensorFwdOp"


def _params(workloads: list[dict]) -> list:
    return [pytest.param(tuple(w["input_shape"]), getattr(torch, d),
                         id=f"{w.get('label', 'manifest')}-{d}")
            for w in workloads for d in w["dtypes"]]


@pytest.mark.parametrize("shape, dtype", _params(load_workloads(_OP)))
def test_lerp_tensor_bench(shape: tuple, dtype: torch.dtype) -> None:
    test = LerpTensorManifestWorkload(shape, dtype)
    inputs = test.gen_inputs()
    op = LerpTensorFwdOp(input=shape, end=shape, weight=shape, dtype=dtype)
    bm = ManifestBenchmark(_OP, op, test)
    result = bm.profile(op, *inputs)
    BenchmarkReport.record(op, locals(), result, tag="tileops")


if __name__ == "__main__":
    pytest.main([__file__, "-vvs"])
