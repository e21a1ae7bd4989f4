"""GatedDeltaNetPrefillFwdOp against the sequential-recurrence oracle.

The reference has no GDN Op or test (it was not delivered); the oracle is the
restated golden_gdn_sequential (examples/gdn_prefill/probe/gdn_prefill_probe.py:60-77).
Output and final state are compared with the half-precision bound
rtol = atol = 1e-2; shapes cover ragged sequence lengths, an initial state,
several heads and, on sampled heads, the full benchmark shape.
"""

import numpy as np
import pytest
import torch

from oracle import tileops_oracle as orc
from tests._util import assert_close_np, to_np
from tileops.kernels.linear_attention.gdn_prefill import GDNPrefillFwdKernel
from tileops.ops.linear_attention import GatedDeltaNetPrefillFwdOp
from tileops.workloads.linear_attention import GdnPrefillWorkload

TOL = 1e-2


def _check(inputs, o, hT, h0, scale, pairs):
    q, k, v, g, beta = (to_np(t) for t in inputs)
    s0 = None if h0 is None else to_np(h0)
    for b, h in pairs:
        sl = (slice(b, b + 1), slice(None), slice(h, h + 1))
        o_ref, h_ref = orc.gdn_sequential(
            q[sl], k[sl], v[sl], g[b:b + 1, :, h:h + 1], beta[b:b + 1, :, h:h + 1],
            None if s0 is None else s0[b:b + 1, h:h + 1], scale,
        )
        assert_close_np(to_np(o)[sl], orc.round_to("bfloat16", o_ref), TOL, TOL, f"o b{b} h{h}")
        assert_close_np(to_np(hT)[b:b + 1, h:h + 1], h_ref, TOL, TOL, f"state b{b} h{h}")


@pytest.mark.gpu
@pytest.mark.parametrize(
    "B, T, H, with_h0",
    [
        pytest.param(1, 64, 1, False, marks=pytest.mark.smoke),
        pytest.param(2, 256, 2, False, marks=pytest.mark.smoke),
        pytest.param(1, 200, 2, True, marks=pytest.mark.full),  # ragged last chunk
        pytest.param(2, 1000, 3, True, marks=pytest.mark.full),
        pytest.param(1, 37, 1, True, marks=pytest.mark.full),   # shorter than a chunk
        # odd chunk counts (the recurrence runs chunks in pairs plus a tail)
        # and workgroup counts that are not a multiple of the 8 XCDs
        pytest.param(1, 130, 2, True, marks=pytest.mark.full),   # 3 chunks, ragged
        pytest.param(2, 320, 1, False, marks=pytest.mark.full),  # 5 chunks
        pytest.param(1, 128, 5, True, marks=pytest.mark.full),   # 2 chunks, 20 workgroups
    ],
)
def test_gdn_prefill_small(B, T, H, with_h0):
    inputs = GdnPrefillWorkload(B, T, H, 128, 128).gen_inputs()
    h0 = torch.randn(B, H, 128, 128, device="cuda") * 0.5 if with_h0 else None
    op = GatedDeltaNetPrefillFwdOp(B, T, H, 128, 128, chunk_size=64)
    o, hT = op(*inputs, initial_state=h0)
    assert o.shape == inputs[2].shape and o.dtype == torch.bfloat16
    assert hT.shape == (B, H, 128, 128) and hT.dtype == torch.float32
    _check(inputs, o, hT, h0, op.scale, [(b, h) for b in range(B) for h in range(H)])


@pytest.mark.gpu
def test_gdn_prefill_benchmark_shape_sampled_heads():
    B, T, H = 4, 8192, 16
    inputs = GdnPrefillWorkload(B, T, H, 128, 128).gen_inputs()
    op = GatedDeltaNetPrefillFwdOp(B, T, H, 128, 128, chunk_size=64)
    o, hT = op(*inputs)
    assert torch.isfinite(o.float()).all() and torch.isfinite(hT).all()
    _check(inputs, o, hT, None, op.scale, [(0, 0), (3, 15), (1, 7)])


@pytest.mark.gpu
def test_gdn_prefill_zero_length_passes_state_through():
    h0 = torch.randn(1, 2, 128, 128, device="cuda")
    e = torch.empty(1, 0, 2, 128, device="cuda", dtype=torch.bfloat16)
    z = torch.empty(1, 0, 2, device="cuda")
    o, hT = GatedDeltaNetPrefillFwdOp(1, 0, 2)(e, e, e, z, z, initial_state=h0)
    assert o.shape == (1, 0, 2, 128)
    torch.testing.assert_close(hT, h0)


@pytest.mark.gpu
def test_gdn_prefill_beta_zero_only_decays():
    B, T, H = 1, 300, 1
    q, k, v, g, beta = GdnPrefillWorkload(B, T, H, 128, 128).gen_inputs()
    beta.zero_()
    h0 = torch.randn(B, H, 128, 128, device="cuda")
    o, hT = GatedDeltaNetPrefillFwdOp(B, T, H)(q, k, v, g, beta, initial_state=h0)
    expect = torch.exp(g.sum(1))[:, :, None, None] * h0
    torch.testing.assert_close(hT, expect, rtol=1e-5, atol=1e-6)


@pytest.mark.smoke
def test_gdn_eval_roofline():
    op = GatedDeltaNetPrefillFwdOp.__new__(GatedDeltaNetPrefillFwdOp)
    op.batch, op.seq_len, op.heads, op.dim_k, op.dim_v = 4, 8192, 16, 128, 128
    op.chunk_size, op.dtype = 64, torch.bfloat16
    assert op.eval_roofline() == (95_205_105_664, 545_259_520)


@pytest.mark.smoke
def test_gdn_kernel_contract():
    with pytest.raises(ValueError, match="only supports dtypes"):
        GDNPrefillFwdKernel(1, 64, 1, 128, 128, 64, torch.float16)
    with pytest.raises(ValueError, match="chunk_size"):
        GDNPrefillFwdKernel(1, 64, 1, 128, 128, 32, torch.bfloat16)
