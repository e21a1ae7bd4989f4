"""FusedAddLayerNormFwdOp against the oracle.

Mirrors tests/ops/test_fused_add_layer_norm.py of the reference (shapes,
tolerances, 3-D input, rejection, roofline, two-output kernel) and adds the
mixed-precision layout (fp32 weight / bias with half activations).
"""

import numpy as np
import pytest
import torch

from oracle import tileops_oracle as orc
from tests._util import NAMES, from_np, ref_tolerance, to_np
from tileops.kernels.norm.fused_add_layer_norm import FusedAddLayerNormKernel
from tileops.ops.norm.fused_add_layer_norm import FusedAddLayerNormFwdOp
from tileops.testing.test_base import TestBase
from tileops.workloads.norm import FusedAddLayerNormWorkload


class FusedAddLayerNormTest(FusedAddLayerNormWorkload, TestBase):
    def ref_program(self, x, residual, weight, bias):
        y, added = orc.fused_add_layer_norm(
            to_np(x), to_np(residual), to_np(weight), to_np(bias), self.eps, NAMES[x.dtype]
        )
        return from_np(y, x), from_np(added, x)


SHAPES = [
    pytest.param(64, 4096, torch.float32, marks=[pytest.mark.smoke, pytest.mark.packaging]),
    pytest.param(64, 4096, torch.float16, marks=pytest.mark.smoke),
    pytest.param(64, 4096, torch.bfloat16, marks=pytest.mark.smoke),
    pytest.param(2048, 4096, torch.float16, marks=pytest.mark.full),
    pytest.param(2048, 4096, torch.bfloat16, marks=pytest.mark.full),
    pytest.param(2048, 5120, torch.float32, marks=pytest.mark.full),
    pytest.param(1025, 4096, torch.float16, marks=pytest.mark.full),
    pytest.param(16, 1152, torch.float16, marks=pytest.mark.smoke),
    pytest.param(8, 8192, torch.bfloat16, marks=pytest.mark.full),
    # one workgroup per row, 5..8 packs per lane (1024 < N / pack <= 2048)
    pytest.param(4, 16384, torch.bfloat16, marks=pytest.mark.full),
    pytest.param(7, 8192, torch.float32, marks=pytest.mark.full),
    pytest.param(9, 12288, torch.float16, marks=pytest.mark.full),
    pytest.param(3, 6148, torch.float32, marks=pytest.mark.full),  # last pack column: 1 lane
    pytest.param(2, 32768, torch.bfloat16, marks=pytest.mark.full),  # beyond registers
    pytest.param(5, 1001, torch.float16, marks=pytest.mark.full),  # odd N: generic path
]


@pytest.mark.gpu
@pytest.mark.parametrize("m, n, dtype", SHAPES)
def test_fused_add_layer_norm_op(m, n, dtype):
    test = FusedAddLayerNormTest(m, n, dtype)
    atol, rtol = ref_tolerance(dtype)
    test.check(FusedAddLayerNormFwdOp(dtype=dtype), *test.gen_inputs(), atol=atol, rtol=rtol)


@pytest.mark.gpu
@pytest.mark.parametrize("param_dtype", [None, torch.float32])
def test_fused_add_layer_norm_many_rows(param_dtype):
    # more rows than the device holds resident workgroups (the persistent
    # path), and a row count that is not a multiple of the rows per
    # workgroup: residual_out bit-exact on every row, y on sampled rows
    m, n, dtype = 12289, 4096, torch.bfloat16
    test = FusedAddLayerNormTest(m, n, dtype, param_dtype=param_dtype)
    x, r, w, b = test.gen_inputs()
    y, r_out = FusedAddLayerNormFwdOp(dtype=dtype)(x, r, w, b)
    assert torch.equal(r_out, (x.float() + r.float()).to(dtype))
    rows = torch.arange(0, m, 97, device=x.device)
    rows = torch.cat([rows, torch.tensor([m - 1], device=x.device)])
    y_ref, _ = test.ref_program(x[rows], r[rows], w, b)
    atol, rtol = ref_tolerance(dtype)
    torch.testing.assert_close(y[rows], y_ref.to(y.device), atol=atol, rtol=rtol)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("n", [4096, 13312])  # wavefront-per-row, workgroup-per-row
def test_fused_add_layer_norm_fp32_params(dtype, n):
    test = FusedAddLayerNormTest(256, n, dtype, param_dtype=torch.float32)
    x, r, w, b = test.gen_inputs()
    assert w.dtype == torch.float32
    op = FusedAddLayerNormFwdOp(dtype=dtype)
    atol, rtol = ref_tolerance(dtype)
    test.check(op, x, r, w, b, atol=atol, rtol=rtol)
    flops, nbytes = op.eval_roofline()
    assert nbytes == 4 * 256 * n * 2 + 2 * n * 4


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_fused_add_layer_norm_3d(dtype):
    x = torch.randn(2, 512, 4096, dtype=dtype, device="cuda")
    r = torch.randn_like(x)
    w = torch.randn(4096, dtype=dtype, device="cuda")
    b = torch.randn(4096, dtype=dtype, device="cuda")
    y, r_out = FusedAddLayerNormFwdOp(dtype=dtype)(x, r, w, b)
    y_ref, added = orc.fused_add_layer_norm(to_np(x), to_np(r), to_np(w), to_np(b), 1e-5,
                                            NAMES[dtype])
    assert y.shape == x.shape and r_out.shape == x.shape
    atol, rtol = ref_tolerance(dtype)
    np.testing.assert_array_equal(to_np(r_out), added)  # rounded sum is exact
    torch.testing.assert_close(torch.from_numpy(to_np(y)), torch.from_numpy(y_ref), atol=atol,
                               rtol=rtol)


@pytest.mark.gpu
def test_fused_add_layer_norm_rejects_bad_shape():
    op = FusedAddLayerNormFwdOp(dtype=torch.float16)
    x = torch.randn(16, 4096, device="cuda", dtype=torch.float16)
    w = torch.randn(4096, device="cuda", dtype=torch.float16)
    with pytest.raises(ValueError, match="residual shape"):
        op(x, x[:, :2048], w, w)


@pytest.mark.gpu
def test_fused_add_layer_norm_kernel_returns_two_outputs():
    test = FusedAddLayerNormTest(8, 4096, torch.float16)
    outputs = FusedAddLayerNormKernel(8, 4096, test.eps, torch.float16)(*test.gen_inputs())
    assert isinstance(outputs, list) and len(outputs) == 2
    assert all(o.shape == (8, 4096) for o in outputs)


@pytest.mark.gpu
def test_fused_add_layer_norm_eval_roofline():
    m, n, dtype = 64, 4096, torch.float16
    op = FusedAddLayerNormFwdOp(dtype=dtype)
    op(*FusedAddLayerNormTest(m, n, dtype).gen_inputs())
    assert op.eval_roofline() == (8 * m * n, (4 * m * n + 2 * n) * 2)


@pytest.mark.smoke
def test_fused_add_layer_norm_kernel_rejects_dtype():
    with pytest.raises(ValueError, match="only supports dtypes"):
        FusedAddLayerNormKernel(4, 8, 1e-5, torch.int32)


@pytest.mark.smoke
def test_fused_add_layer_norm_roofline_needs_forward():
    with pytest.raises(RuntimeError, match="requires a prior"):
        FusedAddLayerNormFwdOp(dtype=torch.float16).eval_roofline()
