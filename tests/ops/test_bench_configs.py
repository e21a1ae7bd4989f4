"""Parity at the exact benchmark configurations (the shapes bench.py times).

Each benchmark input is generated as bench.py generates it and run through
the operator at full size; the result is compared with the oracle:

* Hardswish / Hardsigmoid / ClampScalar(-1, 1), fp16 x[8192, 8192] ~ N(0, 9):
  every element, bit for bit;
* isnan / isinf / isfinite, fp32 x[8192, 8192] with 1% +-inf and 1% NaN at
  seeded random positions: every mask byte (torch.equal);
* GeluAndMul / GeluTanhAndMul, bf16 x[16384, 22016]: 256 sampled rows plus
  the first and last, rtol = atol = 1e-2;
* FusedAddLayerNorm, bf16 [32768, 4096] with fp32 gamma / beta: 256 sampled
  rows (residual_out bit-exact, y at 1e-2);
* LogSumExp and Argmax, fp32 x[32768, 4096] ~ N(0, 4): every row (LSE at the
  fp32 tolerance, indices exact);
* MultiHeadAttentionFwdOp bf16 (8, 4096, 32, 128), causal and non-causal:
  the full output, o and the log2 LSE of 6 sampled (batch, head) pairs plus
  the first and last compared with the fp64 oracle.

GDN prefill at its benchmark shape is in tests/ops/test_gdn_prefill.py.
"""

import numpy as np
import pytest
import torch

from oracle import tileops_oracle as orc
from tests._util import HALF_PRECISION_TOL, assert_bits_equal, assert_close_np, to_np


def _rows(m, n=256, seed=7):
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([[0, m - 1], rng.choice(m, n, replace=False)]))


@pytest.mark.gpu
def test_elementwise_fp16_8192x8192_bit_exact():
    from tileops.ops.elementwise import ClampScalarFwdOp, HardsigmoidFwdOp, HardswishFwdOp
    from tileops.workloads.elementwise import ScaledNormalWorkload

    shape = (8192, 8192)
    n = shape[0] * shape[1]
    (x,) = ScaledNormalWorkload(shape, torch.float16, 3.0).gen_inputs()
    xn = to_np(x)
    for op, ref in ((HardswishFwdOp(n, torch.float16), orc.hardswish(xn, "float16")),
                    (HardsigmoidFwdOp(n, torch.float16), orc.hardsigmoid(xn, "float16")),
                    (ClampScalarFwdOp(n, torch.float16, min=-1.0, max=1.0),
                     orc.clamp_scalar(xn, "float16", -1.0, 1.0))):
        assert_bits_equal(to_np(op(x)), ref, type(op).__name__)


@pytest.mark.gpu
def test_predicates_fp32_8192x8192_exact():
    from tileops.ops.elementwise import IsfiniteFwdOp, IsinfFwdOp, IsnanFwdOp
    from tileops.workloads.elementwise import ScatteredSpecialWorkload

    shape = (8192, 8192)
    n = shape[0] * shape[1]
    (x,) = ScatteredSpecialWorkload(shape, torch.float32).gen_inputs()
    xn = to_np(x)
    assert np.isnan(xn).mean() == pytest.approx(0.01, rel=1e-3)
    for op, ref in ((IsnanFwdOp(n, torch.float32), orc.isnan(xn)),
                    (IsinfFwdOp(n, torch.float32), orc.isinf(xn)),
                    (IsfiniteFwdOp(n, torch.float32), orc.isfinite(xn))):
        y = op(x)
        assert y.dtype == torch.bool
        assert torch.equal(y.cpu(), torch.from_numpy(ref)), type(op).__name__


@pytest.mark.gpu
@pytest.mark.parametrize("approx", ["none", "tanh"])
def test_gated_gelu_bf16_16384x11008(approx):
    from tileops.ops.elementwise import GeluAndMulFwdOp, GeluTanhAndMulFwdOp

    M, N = 16384, 11008
    torch.manual_seed(1235)
    x = torch.randn(M, 2 * N, device="cuda", dtype=torch.bfloat16)
    cls = GeluAndMulFwdOp if approx == "none" else GeluTanhAndMulFwdOp
    y = cls(M, N, torch.bfloat16)(x)
    rows = _rows(M)
    idx = torch.from_numpy(rows).cuda()
    fn = orc.gelu_and_mul if approx == "none" else orc.gelu_tanh_and_mul
    ref = fn(to_np(x.index_select(0, idx)), "bfloat16")
    tol = HALF_PRECISION_TOL
    assert_close_np(to_np(y.index_select(0, idx)), ref, tol, tol, f"gated gelu {approx}")


@pytest.mark.gpu
def test_fused_add_layer_norm_bf16_32768x4096_fp32_params():
    from tileops.ops.norm import FusedAddLayerNormFwdOp
    from tileops.workloads.norm import FusedAddLayerNormWorkload

    wl = FusedAddLayerNormWorkload(32768, 4096, torch.bfloat16, param_dtype=torch.float32)
    x, r, w, b = wl.gen_inputs()
    y, r_out = FusedAddLayerNormFwdOp(dtype=torch.bfloat16, eps=1e-5)(x, r, w, b)
    idx = torch.from_numpy(_rows(32768)).cuda()
    y_ref, added = orc.fused_add_layer_norm(
        to_np(x.index_select(0, idx)), to_np(r.index_select(0, idx)), to_np(w), to_np(b),
        1e-5, "bfloat16")
    assert_bits_equal(to_np(r_out.index_select(0, idx)), added, "residual_out")
    tol = HALF_PRECISION_TOL
    assert_close_np(to_np(y.index_select(0, idx)), y_ref, tol, tol, "layer norm")


@pytest.mark.gpu
def test_logsumexp_argmax_fp32_32768x4096_all_rows():
    from tileops.ops.reduction import ArgmaxFwdOp, LogSumExpFwdOp

    torch.manual_seed(1235)
    x = torch.randn(32768, 4096, device="cuda") * 2.0
    lse = LogSumExpFwdOp(dtype=torch.float32, dim=-1)(x)
    idx = ArgmaxFwdOp(dtype=torch.float32, dim=-1)(x)
    xn = to_np(x)
    assert_close_np(to_np(lse), orc.logsumexp(xn, "float32"), 1e-5, 1e-5, "lse 32768x4096")
    assert torch.equal(idx.cpu(), torch.from_numpy(orc.argreduce(xn, -1)))


@pytest.mark.gpu
@pytest.mark.parametrize("causal", [False, True])
def test_mha_bf16_8x4096x32x128(causal):
    from tileops.ops.attention import MultiHeadAttentionFwdOp

    B, S, H, D = 8, 4096, 32, 128
    torch.manual_seed(1235)
    q, k, v = (torch.randn(B, S, H, D, device="cuda", dtype=torch.bfloat16) for _ in range(3))
    o, lse = MultiHeadAttentionFwdOp(B, H, S, D, causal, torch.bfloat16)(q, k, v)
    rng = np.random.default_rng(3)
    pairs = [(0, 0), (B - 1, H - 1)] + [(int(b), int(h)) for b, h in
                                         zip(rng.integers(0, B, 6), rng.integers(0, H, 6))]
    for b, h in pairs:
        sl = (slice(b, b + 1), slice(None), slice(h, h + 1))
        o_ref, lse_ref = orc.mha_fwd(to_np(q[sl]), to_np(k[sl]), to_np(v[sl]), causal, "bfloat16")
        # atol 5e-3 as the reference test; rows attending to few keys carry
        # |o| ~ 1 where one bf16 ulp is 7.8e-3, hence rtol 1e-2
        assert_close_np(to_np(o[sl]), o_ref, 5e-3, 1e-2, f"o b{b} h{h} causal={causal}")
        assert_close_np(to_np(lse[b:b + 1, h:h + 1]), lse_ref, 1e-3, 1e-4,
                        f"lse b{b} h{h} causal={causal}")
