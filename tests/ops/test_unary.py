"""HardswishFwdOp / HardsigmoidFwdOp / ClampScalarFwdOp against the oracle.

Mirrors tests/ops/test_hardswish.py, test_hardsigmoid.py and
test_clamp_scalar.py of the reference: same parameters, tolerances and
contract checks; ``ref_program`` is the oracle restatement.
"""

import numpy as np
import pytest
import torch

from oracle import tileops_oracle as orc
from tests._util import NAMES, assert_bits_equal, from_np, ref_tolerance, to_np
from tileops.kernels.elementwise.clamp_scalar import ClampScalarFwdKernel
from tileops.kernels.elementwise.hardsigmoid import HardsigmoidFwdKernel
from tileops.kernels.elementwise.hardswish import HardswishFwdKernel
from tileops.ops.elementwise.clamp_scalar import ClampScalarFwdOp
from tileops.ops.elementwise.hardsigmoid import HardsigmoidFwdOp
from tileops.ops.elementwise.hardswish import HardswishFwdOp
from tileops.testing.test_base import TestBase
from tileops.workloads.workload_base import FixtureBase, RandnWorkload

SIZES_DTYPES = [
    pytest.param(1_048_576, torch.float32, marks=[pytest.mark.smoke, pytest.mark.packaging]),
    pytest.param(1_048_576, torch.float16, marks=pytest.mark.smoke),
    pytest.param(1_048_576, torch.bfloat16, marks=pytest.mark.smoke),
    pytest.param(4_000_000, torch.float16, marks=pytest.mark.full),
    pytest.param(4_000_000, torch.bfloat16, marks=pytest.mark.full),
    # ragged: not a multiple of the 16-byte pack, exercises the scalar tail
    pytest.param(1_000_003, torch.float16, marks=pytest.mark.full),
    pytest.param(13, torch.float32, marks=pytest.mark.full),
]


class _UnaryTest(RandnWorkload, TestBase):
    fn = None

    def __init__(self, n_total, dtype, **kw):
        super().__init__((n_total,), dtype)
        self.kw = kw

    def ref_program(self, x):
        return from_np(type(self).fn(to_np(x), NAMES[x.dtype], **self.kw), x)


class HardswishTest(_UnaryTest):
    fn = staticmethod(orc.hardswish)


class HardsigmoidTest(_UnaryTest):
    fn = staticmethod(orc.hardsigmoid)


class ClampTest(_UnaryTest):
    @staticmethod
    def fn(x, dt, min_val=None, max_val=None):
        return orc.clamp_scalar(x, dt, min_val, max_val)


class UnaryFixture(FixtureBase):
    PARAMS = [("n_total, dtype", SIZES_DTYPES)]


@pytest.mark.gpu
@UnaryFixture
def test_hardswish_op(n_total, dtype):
    test = HardswishTest(n_total, dtype)
    atol, rtol = ref_tolerance(dtype)
    test.check(HardswishFwdOp(N_total=n_total, dtype=dtype), *test.gen_inputs(), atol=atol,
               rtol=rtol)


@pytest.mark.gpu
@UnaryFixture
def test_hardsigmoid_op(n_total, dtype):
    test = HardsigmoidTest(n_total, dtype)
    atol, rtol = ref_tolerance(dtype)
    test.check(HardsigmoidFwdOp(N_total=n_total, dtype=dtype), *test.gen_inputs(), atol=atol,
               rtol=rtol)


@pytest.mark.gpu
@UnaryFixture
def test_clamp_scalar_op(n_total, dtype):
    test = ClampTest(n_total, dtype, min_val=-0.5, max_val=0.5)
    atol, rtol = ref_tolerance(dtype)
    op = ClampScalarFwdOp(N_total=n_total, dtype=dtype, min=-0.5, max=0.5)
    test.check(op, *test.gen_inputs(), atol=atol, rtol=rtol)


@pytest.mark.gpu
@pytest.mark.parametrize("min_val, max_val", [(-0.5, 0.5), (None, 0.5), (-0.5, None),
                                              (1.0, -1.0), (float("nan"), 1.0)])
def test_clamp_scalar_param_forms(min_val, max_val):
    test = ClampTest(1024, torch.float32, min_val=min_val, max_val=max_val)
    op = ClampScalarFwdOp(N_total=1024, dtype=torch.float32, min=min_val, max=max_val)
    test.check(op, *test.gen_inputs())


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_activations_all_half_encodings_bitexact(dtype):
    """Every one of the 65,536 encodings (NaN, ±inf, ±0, subnormals included)
    through hardswish and hardsigmoid, bit for bit against the oracle."""
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16)
    x = bits.view(dtype).cuda()
    for op_cls, fn in ((HardswishFwdOp, orc.hardswish), (HardsigmoidFwdOp, orc.hardsigmoid)):
        got = to_np(op_cls(N_total=x.numel(), dtype=dtype)(x))
        assert_bits_equal(got, fn(to_np(x), NAMES[dtype]), f"{op_cls.__name__} {dtype}")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_unary_special_values_bitexact(dtype):
    """Boundary cases of the reference harness (hardswish_fwd_kernel.py:267-337):
    kernels must agree with the oracle bit for bit, NaN and signed zeros included."""
    vals = np.array([0.0, -0.0, -3.0, 3.0, 2.5, -2.5, 6.0, -6.0, 100.0, -100.0, np.nan,
                     np.inf, -np.inf, 1e-30, -1e-30, 0.75], np.float32)
    x = from_np(orc.round_to(NAMES[dtype], vals), torch.empty(0, device="cuda"), dtype)
    for op_cls, fn in ((HardswishFwdOp, orc.hardswish), (HardsigmoidFwdOp, orc.hardsigmoid)):
        got = to_np(op_cls(N_total=x.numel(), dtype=dtype)(x))
        assert_bits_equal(got, fn(to_np(x), NAMES[dtype]), op_cls.__name__)
    for lo, hi in ((-1.0, 1.0), (None, 0.5), (2.0, -2.0), (float("nan"), 1.0)):
        got = to_np(ClampScalarFwdOp(N_total=x.numel(), dtype=dtype, min=lo, max=hi)(x))
        assert_bits_equal(got, orc.clamp_scalar(to_np(x), NAMES[dtype], lo, hi), f"clamp {lo} {hi}")


@pytest.mark.gpu
def test_hardswish_inplace_keeps_identity():
    x = torch.randn(3, 1000, device="cuda", dtype=torch.float16)
    ref = orc.hardswish(to_np(x), "float16")
    op = HardswishFwdOp(N_total=x.numel(), dtype=torch.float16, inplace=True)
    y = op(x)
    assert y is x
    np.testing.assert_array_equal(to_np(x), ref)


@pytest.mark.gpu
def test_unary_keeps_shape_and_handles_noncontiguous():
    x = torch.randn(64, 96, device="cuda", dtype=torch.bfloat16).t()
    y = HardswishFwdOp(N_total=x.numel(), dtype=torch.bfloat16)(x)
    assert y.shape == x.shape
    np.testing.assert_array_equal(to_np(y), orc.hardswish(to_np(x.contiguous()), "bfloat16"))


# -- host-side contract (no GPU) --------------------------------------------------------
@pytest.mark.smoke
@pytest.mark.parametrize("cls", [HardswishFwdKernel, HardsigmoidFwdKernel])
def test_rejects_non_float_dtype(cls):
    with pytest.raises(ValueError, match="only supports dtypes"):
        cls(N_total=16, dtype=torch.int32)


@pytest.mark.smoke
def test_clamp_scalar_kernel_rejects_non_float_dtype():
    with pytest.raises(ValueError, match="only supports dtypes"):
        ClampScalarFwdKernel(N_total=16, dtype=torch.int32, min_val=-0.5)


@pytest.mark.smoke
def test_clamp_scalar_both_none_rejected():
    with pytest.raises(ValueError, match=r"present\(min\) or present\(max\)"):
        ClampScalarFwdOp(N_total=16, dtype=torch.float32, min=None, max=None)


@pytest.mark.smoke
@pytest.mark.parametrize("cls, flops", [(HardswishFwdOp, 4), (HardsigmoidFwdOp, 3)])
def test_activation_eval_roofline(cls, flops):
    N = 1_048_576
    op = cls(N_total=N, dtype=torch.float16)
    assert op.eval_roofline() == (flops * N, 2 * N * 2)


@pytest.mark.smoke
def test_clamp_scalar_eval_roofline():
    N = 1_048_576
    op = ClampScalarFwdOp(N_total=N, dtype=torch.float16, min=-0.5, max=0.5)
    assert op.eval_roofline() == (N, 2 * N * 2)
