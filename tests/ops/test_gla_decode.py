"""GLADecodeOp against the oracle.

Mirrors test_gla_decode.py of the reference: the same cases (fp16 / bf16 /
fp32, DK = DV = 128 serving shapes, non-tile and rectangular shapes, a custom
scale), the same per-dtype tolerances (gla_decode_tolerance), the default
scale and the roofline; the golden is the oracle's restatement of
golden_gla_decode, itself pinned in tests/test_oracle_pins.py.
"""

import pytest
import torch

from oracle import tileops_oracle as orc
from tests._util import NAMES, assert_close_np, to_np
from tileops.kernels.linear_attention.gla_decode import GLADecodeKernel
from tileops.ops.linear_attention.gla_decode import GLADecodeOp
from tileops.workloads.linear_attention import GLADecodeWorkload, gla_decode_tolerance

_F16, _BF16, _F32 = torch.float16, torch.bfloat16, torch.float32

# (B, H, DK, DV, dtype, scale, id) -- the reference's cases, plus DV = 200
# (no 16-byte column groups: the element-wise path) and three shapes of the
# row-slice kernel (16-, 16- over two workgroups, and 4-pack slices), and one
# bf16 and one fp32 whose state exceeds 128 MiB (non-temporal state loads)
_CASES = [
    (2, 4, 64, 64, _F16, -1.0, "smoke-d64-fp16"),
    (2, 4, 64, 64, _BF16, -1.0, "smoke-d64-bf16"),
    (1, 8, 128, 128, _BF16, -1.0, "serving-b1-h8"),
    (1, 32, 128, 128, _BF16, -1.0, "serving-b1-h32"),
    (8, 32, 128, 128, _BF16, -1.0, "serving-b8-h32"),
    (1, 2, 32, 16, _F32, -1.0, "f32-untiled"),
    (2, 3, 16, 16, _F16, -1.0, "small-k16"),
    (1, 4, 128, 64, _F16, -1.0, "rect-d128x64"),
    (2, 3, 64, 64, _BF16, 0.25, "custom-scale"),
    (1, 3, 48, 200, _F16, -1.0, "dv200-elementwise"),
    # the row-slice kernel at its other slice widths and rows per thread
    (2, 3, 256, 256, _BF16, -1.0, "rows-k256-v256"),
    (1, 4, 128, 128, _F32, -1.0, "rows-f32-two-slices"),
    (2, 2, 64, 32, _BF16, -1.0, "rows-4-pack-slices"),
    (64, 66, 128, 128, _BF16, -1.0, "rows-state-over-128MiB"),
    (32, 66, 128, 128, _F32, -1.0, "rows-f32-state-over-128MiB"),
]


@pytest.mark.gpu
@pytest.mark.parametrize("B, H, DK, DV, dtype, scale, case_id",
                         [pytest.param(*c, id=c[-1]) for c in _CASES])
def test_gla_decode(B, H, DK, DV, dtype, scale, case_id):
    test = GLADecodeWorkload(B, H, DK, DV, dtype, scale)
    q, k, v, gk, state = test.gen_inputs()
    op = GLADecodeOp(B, H, DK, DV, scale=scale, dtype=dtype)
    o, ns = op(q, k, v, gk, state)
    assert o.shape == (B, H, DV) and ns.shape == (B, H, DK, DV)
    assert o.dtype == dtype and ns.dtype == dtype
    ref_o, ref_ns = orc.gla_decode(to_np(q), to_np(k), to_np(v), to_np(gk), to_np(state),
                                   test.scale, NAMES[dtype])
    tol = gla_decode_tolerance(dtype)
    assert_close_np(to_np(o), ref_o, tol["atol"], tol["rtol"], f"o {case_id}")
    assert_close_np(to_np(ns), ref_ns, tol["atol"], tol["rtol"], f"new_state {case_id}")


@pytest.mark.gpu
def test_gla_decode_state_is_not_modified_and_steps_chain():
    B, H, DK, DV = 2, 4, 64, 64
    test = GLADecodeWorkload(B, H, DK, DV, _F32)
    q, k, v, gk, state = test.gen_inputs()
    before = state.clone()
    op = GLADecodeOp(B, H, DK, DV, dtype=_F32)
    _, ns1 = op(q, k, v, gk, state)
    assert torch.equal(state, before)
    o2, ns2 = op(q, k, v, gk, ns1)  # a second step from the returned state
    r_o1, r_ns1 = orc.gla_decode(to_np(q), to_np(k), to_np(v), to_np(gk), to_np(state),
                                 test.scale, "float32")
    r_o2, r_ns2 = orc.gla_decode(to_np(q), to_np(k), to_np(v), to_np(gk), r_ns1, test.scale,
                                 "float32")
    assert_close_np(to_np(ns2), r_ns2, 1e-4, 1e-4, "state after two steps")
    assert_close_np(to_np(o2), r_o2, 1e-4, 1e-4, "o of the second step")


@pytest.mark.smoke
def test_gla_decode_default_scale():
    op = GLADecodeOp(1, 2, 64, 64, scale=-1.0, dtype=_F16)
    assert op.kernel.scale == pytest.approx(64**-0.5)
    assert GLADecodeOp(1, 2, 64, 64, scale=0.25, dtype=_F16).kernel.scale == 0.25


@pytest.mark.smoke
def test_gla_decode_eval_roofline():
    B, H, DK, DV = 1, 8, 128, 128
    flops, nbytes = GLADecodeOp(B, H, DK, DV, dtype=_BF16).eval_roofline()
    assert flops == B * H * (5 * DK * DV + DK + DV)
    assert nbytes == B * H * (3 * DK + 2 * DV + 2 * DK * DV) * 2


@pytest.mark.smoke
def test_gla_decode_kernel_contract():
    with pytest.raises(ValueError, match="only supports dtypes"):
        GLADecodeKernel(1, 2, 64, 64, torch.int32)
    with pytest.raises(ValueError, match="DK > 0"):
        GLADecodeKernel(1, 2, 0, 64, _F16)
