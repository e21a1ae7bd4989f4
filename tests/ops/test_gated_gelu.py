"""GeluAndMulFwdOp / GeluTanhAndMulFwdOp against the oracle.

Mirrors tests/ops/test_gelu_and_mul.py and test_gelu_tanh_and_mul.py of the
reference (shapes, tolerances, dtype / shape rejection, roofline, the
constructor-attribute contract of the profiler subprocess).
"""

from math import prod

import pytest
import torch

from oracle import tileops_oracle as orc
from tests._util import NAMES, from_np, to_np
from tileops.benchmark.rocprof import _extract_op_init_args
from tileops.kernels.elementwise.gelu_and_mul import GeluAndMulFwdKernel
from tileops.kernels.elementwise.gelu_tanh_and_mul import GeluTanhAndMulFwdKernel
from tileops.ops.elementwise.gelu_and_mul import GeluAndMulFwdOp
from tileops.ops.elementwise.gelu_tanh_and_mul import GeluTanhAndMulFwdOp
from tileops.testing.test_base import TestBase
from tileops.workloads.elementwise import GeluAndMulWorkload

OPS = {"erf": (GeluAndMulFwdOp, orc.gelu_and_mul), "tanh": (GeluTanhAndMulFwdOp, orc.gelu_tanh_and_mul)}


def _tol(dtype):
    # tests/ops/test_gelu_and_mul.py:35-42
    if dtype == torch.float32:
        return 1e-5, 1e-5
    if dtype == torch.float16:
        return 1e-2, 1e-2
    return 1.6e-2, 1.6e-2


class GatedTest(GeluAndMulWorkload, TestBase):
    def __init__(self, form, M, N, dtype):
        super().__init__(M, N, dtype)
        self.form = form

    def ref_program(self, x):
        return from_np(OPS[self.form][1](to_np(x), NAMES[x.dtype]), x)


@pytest.mark.gpu
@pytest.mark.parametrize("form", list(OPS))
@pytest.mark.parametrize(
    "M, N, dtype",
    [
        pytest.param(16, 128, torch.float32, marks=[pytest.mark.smoke, pytest.mark.packaging]),
        pytest.param(16, 128, torch.float16, marks=pytest.mark.smoke),
        pytest.param(16, 128, torch.bfloat16, marks=pytest.mark.smoke),
        pytest.param(2048, 14336, torch.float16, marks=pytest.mark.full),
        pytest.param(2048, 14336, torch.bfloat16, marks=pytest.mark.full),
        pytest.param(1, 14336, torch.bfloat16, marks=pytest.mark.full),
        pytest.param(7, 1001, torch.bfloat16, marks=pytest.mark.full),  # odd N: scalar path
        pytest.param(5, 36, torch.float32, marks=pytest.mark.full),
    ],
)
def test_gated_gelu_op(form, M, N, dtype):
    test = GatedTest(form, M, N, dtype)
    atol, rtol = _tol(dtype)
    test.check(OPS[form][0](M=M, N=N, dtype=dtype), *test.gen_inputs(), atol=atol, rtol=rtol)


@pytest.mark.gpu
@pytest.mark.parametrize("form", list(OPS))
def test_gated_gelu_extreme_gates(form):
    M, N = 4, 64
    x = torch.zeros(M, 2 * N, device="cuda", dtype=torch.float32)
    x[:, :N] = torch.linspace(-30, 30, N, device="cuda")
    x[:, N:] = 1.5
    y = OPS[form][0](M=M, N=N, dtype=torch.float32)(x)
    ref = OPS[form][1](to_np(x), "float32")
    torch.testing.assert_close(to_np(y), ref, atol=1e-5, rtol=1e-5, check_dtype=False)


@pytest.mark.smoke
@pytest.mark.parametrize("form", list(OPS))
def test_gated_gelu_rejects_non_float_dtype(form):
    with pytest.raises(ValueError, match="does not support dtype"):
        OPS[form][0](M=16, N=16, dtype=torch.int32)
    kcls = GeluAndMulFwdKernel if form == "erf" else GeluTanhAndMulFwdKernel
    with pytest.raises(ValueError, match="only supports dtypes"):
        kcls(M=16, N=16, dtype=torch.int32)


@pytest.mark.gpu
@pytest.mark.parametrize("form", list(OPS))
def test_gated_gelu_rejects_mismatch(form):
    op = OPS[form][0](M=4, N=8, dtype=torch.float32)
    with pytest.raises(ValueError, match="x.dtype"):
        op(torch.randn(4, 16, device="cuda", dtype=torch.float16))
    with pytest.raises(ValueError, match="x.shape"):
        op(torch.randn(4, 18, device="cuda", dtype=torch.float32))


@pytest.mark.smoke
@pytest.mark.parametrize("form, flops", [("erf", 6), ("tanh", 10)])
def test_gated_gelu_eval_roofline(form, flops):
    M, N = 64, 128
    op = OPS[form][0](M=M, N=N, dtype=torch.float16)
    assert op.eval_roofline() == (flops * M * N, 3 * M * N * 2)
    assert op.N_total == M * N and prod(op.out_shape) == M * N
    assert _extract_op_init_args(op) == {"M": M, "N": N, "dtype": torch.float16}
