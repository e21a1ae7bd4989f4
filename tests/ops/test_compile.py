"""The torch.compile contract of the custom-op Ops.

The reference wraps each kernel in a torch custom op with a fake (meta)
implementation, so that an Op traces into one graph
(examples/TileOPs/tileops/manifest/attention.yaml:19 names
``MultiHeadAttentionFwdOp`` as compile-traced).  Here each Op is compiled
with ``fullgraph=True`` (any graph break fails the test) under the
``aot_eager`` backend, which runs the traced graph through the fake
implementations for shapes and dtypes and then through the real kernels,
and its outputs must equal the eager call's bit for bit.
"""

import pytest
import torch

from tileops.ops.attention.multi_head_attention import MultiHeadAttentionFwdOp
from tileops.ops.linear_attention import GatedDeltaNetDecodeFwdOp
from tileops.ops.reduction.argmax import ArgmaxFwdOp
from tileops.ops.reduction.softmax import LogSumExpFwdOp


def _compiled(op):
    torch._dynamo.reset()
    return torch.compile(op, fullgraph=True, backend="aot_eager")


@pytest.mark.gpu
@pytest.mark.parametrize("causal", [False, True])
def test_mha_compiles_to_one_graph(causal):
    B, H, S, D = 2, 4, 640, 128
    gen = torch.Generator().manual_seed(11)
    q, k, v = (torch.randn(B, S, H, D, generator=gen).bfloat16().cuda() for _ in range(3))
    op = MultiHeadAttentionFwdOp(B, H, S, D, causal, torch.bfloat16)
    o_e, lse_e = op(q, k, v)
    o_c, lse_c = _compiled(op)(q, k, v)
    assert o_c.shape == o_e.shape and o_c.dtype == o_e.dtype
    assert lse_c.shape == lse_e.shape and lse_c.dtype == lse_e.dtype
    assert torch.equal(o_c, o_e) and torch.equal(lse_c, lse_e)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_logsumexp_compiles_to_one_graph(dtype):
    x = (torch.randn(96, 1000, generator=torch.Generator().manual_seed(12)) * 2).to(dtype).cuda()
    op = LogSumExpFwdOp(dtype=dtype, dim=-1)
    y_e = op(x)
    y_c = _compiled(op)(x)
    assert y_c.shape == y_e.shape and y_c.dtype == y_e.dtype
    assert torch.equal(y_c, y_e)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_argmax_compiles_to_one_graph(dtype):
    x = torch.randn(64, 3000, generator=torch.Generator().manual_seed(13)).to(dtype).cuda()
    x[3, 17] = float("nan")  # NaN wins, first occurrence
    op = ArgmaxFwdOp(dtype=dtype, dim=-1)
    i_e = op(x)
    i_c = _compiled(op)(x)
    assert i_c.shape == i_e.shape and i_c.dtype == i_e.dtype
    assert torch.equal(i_c, i_e)


@pytest.mark.gpu
def test_gdn_decode_compiles_to_one_graph():
    B, H, K, V = 2, 4, 128, 64
    gen = torch.Generator().manual_seed(14)
    q, k = (torch.nn.functional.normalize(torch.randn(B, H, K, generator=gen), dim=-1)
            .bfloat16().cuda() for _ in range(2))
    v = torch.randn(B, H, V, generator=gen).bfloat16().cuda()
    g = torch.nn.functional.logsigmoid(torch.randn(B, H, generator=gen)).cuda()
    beta = torch.sigmoid(torch.randn(B, H, generator=gen)).cuda()
    state = torch.randn(B, H, K, V, generator=gen).cuda()
    op = GatedDeltaNetDecodeFwdOp(B, H, K, V)
    o_e, s_e = op(q, k, v, g, beta, state)
    o_c, s_c = _compiled(op)(q, k, v, g, beta, state)
    assert o_c.dtype == o_e.dtype and s_c.dtype == s_e.dtype
    assert torch.equal(o_c, o_e) and torch.equal(s_c, s_e)
