"""IsnanFwdOp / IsinfFwdOp / IsfiniteFwdOp: bool masks bit-exact against the oracle.

Mirrors tests/ops/test_isnan.py, test_isinf.py and test_isfinite.py of the
reference (quarter NaN / +inf / -inf draw, exact comparison, contract tests)
and adds the scattered 1% +-inf / 1% NaN draw and exhaustive half encodings.
"""

import numpy as np
import pytest
import torch

from oracle import tileops_oracle as orc
from tests._util import to_np
from tileops.kernels.elementwise.isfinite import IsfiniteFwdKernel
from tileops.kernels.elementwise.isinf import IsinfFwdKernel
from tileops.kernels.elementwise.isnan import IsnanFwdKernel
from tileops.ops.elementwise.isfinite import IsfiniteFwdOp
from tileops.ops.elementwise.isinf import IsinfFwdOp
from tileops.ops.elementwise.isnan import IsnanFwdOp
from tileops.testing.test_base import TestBase, exact_compare
from tileops.workloads.elementwise import IsnanWorkload, ScatteredSpecialWorkload

OPS = {"isnan": IsnanFwdOp, "isinf": IsinfFwdOp, "isfinite": IsfiniteFwdOp}
KERNELS = {"isnan": IsnanFwdKernel, "isinf": IsinfFwdKernel, "isfinite": IsfiniteFwdKernel}


class PredicateTest(IsnanWorkload, TestBase):
    def __init__(self, name, n_total, dtype):
        super().__init__((n_total,), dtype)
        self.name = name

    def ref_program(self, x):
        return torch.from_numpy(getattr(orc, self.name)(to_np(x))).to(x.device)


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(OPS))
@pytest.mark.parametrize(
    "n_total, dtype",
    [
        pytest.param(1_048_576, torch.float32, marks=pytest.mark.smoke),
        pytest.param(1_048_576, torch.float16, marks=pytest.mark.smoke),
        pytest.param(1_048_576, torch.bfloat16, marks=pytest.mark.smoke),
        pytest.param(4_000_000, torch.float16, marks=pytest.mark.full),
        pytest.param(4_000_000, torch.bfloat16, marks=pytest.mark.full),
        pytest.param(1_000_007, torch.float32, marks=pytest.mark.full),  # ragged tail
    ],
)
def test_predicate_op(name, n_total, dtype):
    test = PredicateTest(name, n_total, dtype)
    test.check(OPS[name](N_total=n_total, dtype=dtype), *test.gen_inputs(), compare=exact_compare)


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(OPS))
def test_predicate_scattered_specials(name):
    (x,) = ScatteredSpecialWorkload((2048, 1024), torch.float32).gen_inputs()
    y = OPS[name](N_total=x.numel(), dtype=torch.float32)(x)
    assert y.dtype == torch.bool and y.shape == x.shape
    np.testing.assert_array_equal(to_np(y), getattr(orc, name)(to_np(x)))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_predicates_exhaustive_half_encodings(dtype):
    x = torch.arange(1 << 16, dtype=torch.int32).to(torch.int16).view(dtype).cuda()
    for name, op in OPS.items():
        got = to_np(op(N_total=x.numel(), dtype=dtype)(x))
        np.testing.assert_array_equal(got, getattr(torch, name)(x.cpu()).numpy(), err_msg=name)


@pytest.mark.gpu
def test_predicate_fp32_encodings():
    enc = np.array([0x7F800000, 0xFF800000, 0x7F800001, 0xFFC00000, 0x7FC00000, 0x7FFFFFFF,
                    0x00000001, 0x80000000, 0x7F7FFFFF, 0x3F800000] * 4, np.uint32)
    x = torch.from_numpy(enc.view(np.float32).copy()).cuda()
    for name, op in OPS.items():
        got = to_np(op(N_total=x.numel(), dtype=torch.float32)(x))
        np.testing.assert_array_equal(got, getattr(orc, name)(to_np(x)), err_msg=name)


@pytest.mark.gpu
def test_isnan_output_dtype_and_values():
    n = 4096
    x = torch.randn(n, device="cuda")
    x[: n // 2] = float("nan")
    y = IsnanFwdOp(N_total=n, dtype=torch.float32)(x)
    assert y.dtype == torch.bool and tuple(y.shape) == (n,)
    assert bool(y[: n // 2].all()) and not bool(y[n // 2 :].any())


@pytest.mark.smoke
@pytest.mark.parametrize("name", list(OPS))
def test_predicate_rejects_non_float_dtype(name):
    with pytest.raises(ValueError, match="only supports dtypes"):
        KERNELS[name](N_total=16, dtype=torch.int32)
    with pytest.raises(ValueError, match="does not support dtype"):
        OPS[name](N_total=16, dtype=torch.int32)


@pytest.mark.smoke
@pytest.mark.parametrize("name", list(OPS))
def test_predicate_eval_roofline(name):
    N = 1_048_576
    op = OPS[name](N_total=N, dtype=torch.float16)
    assert op.eval_roofline() == (N, N * (2 + 1))
