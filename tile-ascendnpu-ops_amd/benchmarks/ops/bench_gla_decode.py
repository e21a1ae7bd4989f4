"""Benchmarks of GLADecodeOp over its manifest workloads (reference bench file:
examples/TileOPs/benchmarks/ops/bench_gla_decode.py)."""

import pytest
import torch

from tileops.benchmark.benchmark_base import BenchmarkReport, ManifestBenchmark
from tileops.manifest import load_workloads
from tileops.ops.linear_attention.gla_decode import GLADecodeOp
from tileops.workloads.linear_attention import GLADecodeWorkload

_OP = "GLADecodeOp"


def _params(workloads: list[dict]) -> list:
    return [pytest.param(w["B"], w["H"], w["DK"], w["DV"], w.get("scale", -1.0),
                         getattr(torch, d), id=f"{w.get('label', 'manifest')}-{d}")
            for w in workloads for d in w["dtypes"]]


@pytest.mark.parametrize("B, H, DK, DV, scale, dtype", _params(load_workloads(_OP)))
def test_gla_decode_bench(B: int, H: int, DK: int, DV: int, scale: float,
                          dtype: torch.dtype) -> None:
    test = GLADecodeWorkload(B, H, DK, DV, dtype, scale)
    inputs = test.gen_inputs()
    op = GLADecodeOp(B, H, DK, DV, scale=scale, dtype=dtype)
    bm = ManifestBenchmark(_OP, op, test)
    result = bm.profile(op, *inputs)
    BenchmarkReport.record(op, locals(), result, tag="tileops")


if __name__ == "__main__":
    pytest.main([__file__, "-vvs"])
