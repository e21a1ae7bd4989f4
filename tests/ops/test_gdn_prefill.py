"""GatedDeltaNetPrefillFwdOp against the sequential-recurrence oracle.

The reference has no GDN Op or test (it was not delivered); the oracle is the
restated golden_gdn_sequential (examples/gdn_prefill/probe/gdn_prefill_probe.py:60-77).
The bf16 output o is compared with the half-precision bound rtol = atol =
1e-2.  The fp32 final state, every product of which takes bf16 operands (as
the reference's chunked form does), is compared at rtol = atol = 5e-3 (the
largest error recorded over these cases is 0.19 of 1e-2), and at 1e-2 under
slow decay, where the state carries across a thousand tokens and several
composed segment maps (largest recorded error 0.54 of 1e-2).  Every check
prints the largest error of o and of the state as a fraction of its bound,
so that the margin is on record in the test log.  Shapes cover ragged sequence lengths,
an initial state, several heads, forced segment counts (the sequence split
into segments whose state maps are composed) with slow decay, so that the
maps carry the state across many chunks, and, on sampled heads, the full
benchmark shape.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import tileops_oracle as orc
from tests._util import assert_close_np, to_np
from tileops.kernels.linear_attention.gdn_prefill import GDNPrefillFwdKernel
from tileops.ops.linear_attention import GatedDeltaNetPrefillFwdOp
from tileops.workloads.linear_attention import GdnPrefillWorkload

TOL = 1e-2  # o (bf16), and the state under slow decay
STATE_TOL = 5e-3  # the fp32 state at the workload's decay


def _frac(got, ref, tol=TOL):
    """Largest |got - ref| / (tol + tol |ref|): 1.0 is the bound."""
    return float(np.max(np.abs(got - ref) / (tol + tol * np.abs(ref)))) if ref.size else 0.0


def _check(inputs, o, hT, h0, scale, pairs, label="", state_tol=STATE_TOL):
    q, k, v, g, beta = (to_np(t) for t in inputs)
    s0 = None if h0 is None else to_np(h0)
    worst_o = worst_s = 0.0
    for b, h in pairs:
        sl = (slice(b, b + 1), slice(None), slice(h, h + 1))
        o_ref, h_ref = orc.gdn_sequential(
            q[sl], k[sl], v[sl], g[b:b + 1, :, h:h + 1], beta[b:b + 1, :, h:h + 1],
            None if s0 is None else s0[b:b + 1, h:h + 1], scale,
        )
        o_ref = orc.round_to("bfloat16", o_ref)
        got_o, got_s = to_np(o)[sl], to_np(hT)[b:b + 1, h:h + 1]
        worst_o = max(worst_o, _frac(got_o, o_ref))
        worst_s = max(worst_s, _frac(got_s, h_ref, state_tol))
        assert_close_np(got_o, o_ref, TOL, TOL, f"o b{b} h{h}")
        assert_close_np(got_s, h_ref, state_tol, state_tol, f"state b{b} h{h}")
    print(f"[gdn {label}] largest error / bound: o {worst_o:.3f}, state {worst_s:.3f}")
    return worst_o, worst_s


def _slow_inputs(B, T, H, seed):
    """Workload inputs with the log-decay scaled by 1/100: the state lives for
    thousands of tokens, so every segment map matters."""
    gen = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(B, T, H, 128, generator=gen), dim=-1).bfloat16()
    k = F.normalize(torch.randn(B, T, H, 128, generator=gen), dim=-1).bfloat16()
    v = torch.randn(B, T, H, 128, generator=gen).bfloat16()
    g = F.logsigmoid(torch.randn(B, T, H, generator=gen)) * 0.01
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen))
    return tuple(t.cuda() for t in (q, k, v, g, beta))


@pytest.mark.gpu
@pytest.mark.parametrize(
    "B, T, H, with_h0",
    [
        pytest.param(1, 64, 1, False, marks=pytest.mark.smoke),
        pytest.param(2, 256, 2, False, marks=pytest.mark.smoke),
        pytest.param(1, 200, 2, True, marks=pytest.mark.full),  # ragged last chunk
        pytest.param(2, 1000, 3, True, marks=pytest.mark.full),
        pytest.param(1, 37, 1, True, marks=pytest.mark.full),   # shorter than a chunk
        pytest.param(1, 1, 2, True, marks=pytest.mark.full),    # a single token
        pytest.param(2, 65, 3, True, marks=pytest.mark.full),   # a chunk and one token
        pytest.param(1, 130, 2, True, marks=pytest.mark.full),   # 3 chunks, ragged
        pytest.param(2, 320, 1, False, marks=pytest.mark.full),  # 5 chunks
        pytest.param(1, 128, 5, True, marks=pytest.mark.full),   # 2 chunks, 5 heads
        pytest.param(3, 1500, 11, True, marks=pytest.mark.full),  # 33 heads, several segments
    ],
)
def test_gdn_prefill_small(B, T, H, with_h0):
    inputs = GdnPrefillWorkload(B, T, H, 128, 128).gen_inputs()
    h0 = torch.randn(B, H, 128, 128, device="cuda") * 0.5 if with_h0 else None
    op = GatedDeltaNetPrefillFwdOp(B, T, H, 128, 128, chunk_size=64)
    o, hT = op(*inputs, initial_state=h0)
    assert o.shape == inputs[2].shape and o.dtype == torch.bfloat16
    assert hT.shape == (B, H, 128, 128) and hT.dtype == torch.float32
    pairs = [(b, h) for b in range(B) for h in range(H)][:12]
    _check(inputs, o, hT, h0, op.scale, pairs, f"B{B} T{T} H{H}")


@pytest.mark.gpu
@pytest.mark.parametrize(
    "B, T, H, segments, with_h0",
    [
        (1, 1024, 1, 2, False),   # two segments: no map, composition from the first
        (1, 1024, 1, 3, True),    # one map
        (1, 1300, 2, 5, True),    # three maps, ragged last chunk
        (1, 1100, 1, 16, True),   # sixteen segments of one or two chunks
        (2, 700, 1, 11, False),   # eleven segments, 11 chunks (one each)
        (2, 1100, 4, 5, True),    # 8 heads: the composition's XCD-grouped workgroups, every head
    ],
)
def test_gdn_prefill_segments_with_slow_decay(B, T, H, segments, with_h0):
    inputs = _slow_inputs(B, T, H, 1000 + T + segments)
    h0 = (torch.randn(B, H, 128, 128, generator=torch.Generator().manual_seed(7)) * 0.5).cuda() \
        if with_h0 else None
    kern = GDNPrefillFwdKernel(B, T, H, 128, 128, 64, torch.bfloat16,
                               config={"segments": segments})
    o, hT = kern(*inputs, h0)
    _check(inputs, o, hT, h0, 128**-0.5, [(b, h) for b in range(B) for h in range(H)],
           f"B{B} T{T} H{H} {segments} segments, slow decay", state_tol=TOL)
    # one segment (no maps) agrees within the same bound
    o1, hT1 = GDNPrefillFwdKernel(B, T, H, 128, 128, 64, torch.bfloat16,
                                  config={"segments": 1})(*inputs, h0)
    assert_close_np(to_np(o), to_np(o1), TOL, TOL, "o, segmented vs one segment")
    assert_close_np(to_np(hT), to_np(hT1), TOL, TOL, "state, segmented vs one segment")


@pytest.mark.gpu
def test_gdn_prefill_benchmark_shape_sampled_heads():
    B, T, H = 4, 8192, 16
    inputs = GdnPrefillWorkload(B, T, H, 128, 128).gen_inputs()
    op = GatedDeltaNetPrefillFwdOp(B, T, H, 128, 128, chunk_size=64)
    o, hT = op(*inputs)
    assert torch.isfinite(o.float()).all() and torch.isfinite(hT).all()
    # heads of every segment position of the launch order
    _check(inputs, o, hT, None, op.scale, [(0, 0), (3, 15), (1, 7), (2, 3), (0, 9), (3, 1)],
           "B4 T8192 H16")


@pytest.mark.gpu
def test_gdn_prefill_zero_length_passes_state_through():
    h0 = torch.randn(1, 2, 128, 128, device="cuda")
    e = torch.empty(1, 0, 2, 128, device="cuda", dtype=torch.bfloat16)
    z = torch.empty(1, 0, 2, device="cuda")
    o, hT = GatedDeltaNetPrefillFwdOp(1, 0, 2)(e, e, e, z, z, initial_state=h0)
    assert o.shape == (1, 0, 2, 128)
    torch.testing.assert_close(hT, h0)


@pytest.mark.gpu
@pytest.mark.parametrize("segments", [1, 3])
def test_gdn_prefill_beta_zero_only_decays(segments):
    B, T, H = 1, 1300, 1
    q, k, v, g, beta = GdnPrefillWorkload(B, T, H, 128, 128).gen_inputs()
    g = g * 0.001  # the state survives the sequence
    beta.zero_()
    h0 = torch.randn(B, H, 128, 128, device="cuda")
    kern = GDNPrefillFwdKernel(B, T, H, 128, 128, 64, torch.bfloat16,
                               config={"segments": segments})
    o, hT = kern(q, k, v, g, beta, h0)
    expect = torch.exp(g.sum(1))[:, :, None, None] * h0
    # the segmented run composes the decay through bf16-split map products
    tol = 1e-5 if segments == 1 else 1e-4
    torch.testing.assert_close(hT, expect, rtol=tol, atol=tol)


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
