"""Benchmarks of GatedDeltaNetDecodeFwdOp over its manifest workloads (no
reference counterpart: the reference has no GDN Op)."""

import pytest
import torch

from tileops.benchmark.benchmark_base import BenchmarkReport, ManifestBenchmark
from tileops.manifest import load_workloads
from tileops.ops.linear_attention.gdn_decode import GatedDeltaNetDecodeFwdOp
from tileops.workloads.linear_attention import GdnDecodeWorkload

_OP = "GatedDeltaNetDecodeFwdOp"


def _params(workloads: list[dict]) -> list:
    return [pytest.param(w["batch"], w["heads"], w["dim_k"], w["dim_v"], getattr(torch, d),
                         id=f"{w.get('label', 'manifest')}-{d}")
            for w in workloads for d in w["dtypes"]]


@pytest.mark.parametrize("batch, heads, dim_k, dim_v, dtype", _params(load_workloads(_OP)))
def test_gdn_decode_bench(batch: int, heads: int, dim_k: int, dim_v: int,
                          dtype: torch.dtype) -> None:
    test = GdnDecodeWorkload(batch, heads, dim_k, dim_v, dtype)
    inputs = test.gen_inputs()
    op = GatedDeltaNetDecodeFwdOp(batch, heads, dim_k, dim_v, dtype=dtype)
    bm = ManifestBenchmark(_OP, op, test)
    result = bm.profile(op, *inputs)
    BenchmarkReport.record(op, locals(), result, tag="tileops")


if __name__ == "__main__":
    pytest.main([__file__, "-vvs"])
