"""Benchmarks of MultiHeadAttentionFwdOp over its manifest workloads
(reference bench file: examples/TileOPs/benchmarks/ops/bench_multi_head_attention.py).
Three tensor inputs, so the rows are expanded here rather than through
``workloads_to_params``."""

import pytest
import torch

from tileops.benchmark.benchmark_base import BenchmarkReport, ManifestBenchmark
from tileops.manifest import load_workloads
from tileops.ops.attention.multi_head_attention import MultiHeadAttentionFwdOp
from tileops.workloads.attention import MhaFwdWorkload

_OP = "MultiHeadAttentionFwdOp"


def _params(workloads: list[dict]) -> list:
    out = []
    for w in workloads:
        batch, seq_len, heads, dim = w["q_shape"]
        marks = (pytest.mark.skip(reason=w["bench_skip_reason"]),) if w.get("bench_skip_reason") else ()
        out += [pytest.param(batch, seq_len, heads, dim, w.get("is_causal", True), getattr(torch, d),
                             id=f"{w.get('label', 'manifest')}-{d}", marks=marks)
                for d in w["dtypes"]]
    return out


@pytest.mark.parametrize("batch, seq_len, heads, dim, causal, dtype", _params(load_workloads(_OP)))
def test_mha_fwd_bench(batch: int, seq_len: int, heads: int, dim: int, causal: bool,
                       dtype: torch.dtype) -> None:
    test = MhaFwdWorkload(batch, heads, seq_len, dim, causal, dtype)
    inputs = test.gen_inputs()
    op = MultiHeadAttentionFwdOp(batch, heads, seq_len, dim, causal, dtype)
    bm = ManifestBenchmark(_OP, op, test)
    result = bm.profile(op, *inputs)
    BenchmarkReport.record(op, locals(), result, tag="tileops")


if __name__ == "__main__":
    pytest.main([__file__, "-vvs"])
