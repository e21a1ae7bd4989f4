"""Benchmarks of FusedAddLayerNormFwdOp over its manifest workloads
(reference bench file: examples/TileOPs/benchmarks/ops/bench_fused_add_layer_norm.py).
A row's ``param_dtype`` (fp32 weight / bias) is honoured."""

import pytest
import torch

from tileops.benchmark.benchmark_base import BenchmarkReport, ManifestBenchmark
from tileops.manifest import load_workloads
from tileops.ops.norm.fused_add_layer_norm import FusedAddLayerNormFwdOp
from tileops.workloads.norm import FusedAddLayerNormWorkload

_OP = "FusedAddLayerNormFwdOp"


def _params(workloads: list[dict]) -> list:
    out = []
    for w in workloads:
        *lead, n = w["x_shape"]
        m = 1
        for s in lead:
            m *= s
        pd = getattr(torch, w["param_dtype"]) if w.get("param_dtype") else None
        out += [pytest.param(m, n, getattr(torch, d), pd, id=f"{w.get('label', 'manifest')}-{d}")
                for d in w["dtypes"]]
    return out


@pytest.mark.parametrize("m, n, dtype, param_dtype", _params(load_workloads(_OP)))
def test_fused_add_layer_norm_bench(m: int, n: int, dtype: torch.dtype, param_dtype) -> None:
    test = FusedAddLayerNormWorkload(m, n, dtype, param_dtype=param_dtype)
    inputs = test.gen_inputs()
    op = FusedAddLayerNormFwdOp(M=m, N=n, dtype=dtype)
    bm = ManifestBenchmark(_OP, op, test)
    result = bm.profile(op, *inputs)
    BenchmarkReport.record(op, locals(), result, tag="tileops")


if __name__ == "__main__":
    pytest.main([__file__, "-vvs"])
