"""LogSumExpFwdOp and ArgmaxFwdOp against the oracle.

Mirrors tests/ops/test_softmax.py (LogSumExp subset) and tests/ops/test_argmax.py
of the reference: shapes, dims, keepdim, dim=None, non-contiguous input, the
multidim rejection, roofline; argmax indices compared exactly (torch.equal).
Adds special-value rows (all -inf, +inf, NaN, ties, signed zeros).
"""

import numpy as np
import pytest
import torch

from oracle import tileops_oracle as orc
from tests._util import NAMES, assert_close_np, from_np, ref_tolerance, to_np
from tileops.kernels.reduction.argmax import ArgreduceKernel
from tileops.kernels.reduction.logsumexp import LogSumExpKernel
from tileops.ops.reduction.argmax import ArgmaxFwdOp
from tileops.ops.reduction.softmax import LogSumExpFwdOp
from tileops.testing.test_base import TestBase
from tileops.workloads.reduction import ArgmaxWorkload, LogSumExpWorkload


def _exact_compare(output, output_ref):
    assert output.dtype == torch.int64 and output_ref.dtype == torch.int64
    assert torch.equal(output, output_ref.to(output.device)), (
        f"mismatches: {(output.cpu() != output_ref.cpu()).sum().item()} / {output.numel()}"
    )


def _lse_ref(x, dim, keepdim=False):
    a = to_np(x)
    dims = [dim] if isinstance(dim, int) else list(dim)
    dims = sorted(d % a.ndim for d in dims)
    kept = [i for i in range(a.ndim) if i not in dims]
    flat = np.transpose(a, kept + dims).reshape([a.shape[i] for i in kept] + [-1])
    y = orc.logsumexp(flat, NAMES[x.dtype])
    if keepdim:
        shape = list(a.shape)
        for d in dims:
            shape[d] = 1
        y = y.reshape(shape)
    return y


class LogSumExpTest(LogSumExpWorkload, TestBase):
    def __init__(self, shape, dtype, dim=-1):
        super().__init__(shape, dtype)
        self.dim = dim

    def ref_program(self, x):
        return from_np(np.asarray(_lse_ref(x, self.dim)), x)


@pytest.mark.gpu
@pytest.mark.parametrize(
    "shape, dim, dtype",
    [
        pytest.param((32, 256), -1, torch.float32, marks=[pytest.mark.smoke]),
        pytest.param((32, 256), -1, torch.float16, marks=pytest.mark.smoke),
        pytest.param((32, 256), -1, torch.bfloat16, marks=pytest.mark.smoke),
        pytest.param((32, 300), -1, torch.float32, marks=pytest.mark.full),
        pytest.param((32, 300), -1, torch.float16, marks=pytest.mark.full),
        pytest.param((32, 300), -1, torch.bfloat16, marks=pytest.mark.full),
        pytest.param((33, 256), -1, torch.float32, marks=pytest.mark.full),
        pytest.param((2, 16, 256), -1, torch.float16, marks=pytest.mark.full),
        pytest.param((4, 32768), -1, torch.float16, marks=pytest.mark.full),
        pytest.param((4, 102400), -1, torch.bfloat16, marks=pytest.mark.full),
        pytest.param((256, 32), 0, torch.float32, marks=pytest.mark.full),
        pytest.param((256, 32), 0, torch.float16, marks=pytest.mark.full),
        pytest.param((8192, 4096), -1, torch.float32, marks=pytest.mark.full),
        pytest.param((4000, 131), -1, torch.float32, marks=pytest.mark.full),
    ],
)
def test_logsumexp_op(shape, dim, dtype):
    test = LogSumExpTest(shape, dtype, dim=dim)
    atol, rtol = ref_tolerance(dtype)
    test.check(LogSumExpFwdOp(dtype=dtype, dim=dim), *test.gen_inputs(), atol=atol, rtol=rtol)


@pytest.mark.gpu
@pytest.mark.parametrize("shape, dim, dtype", [((32, 256), -1, torch.float32),
                                               ((256, 32), 0, torch.float16)])
def test_logsumexp_keepdim(shape, dim, dtype):
    x = torch.randn(*shape, dtype=dtype, device="cuda")
    y = LogSumExpFwdOp(dtype=dtype, dim=dim, keepdim=True)(x)
    ref = _lse_ref(x, dim, keepdim=True)
    assert tuple(y.shape) == ref.shape
    atol, rtol = ref_tolerance(dtype)
    assert_close_np(to_np(y), ref, atol, rtol, "lse keepdim")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_logsumexp_1d_and_multidim(dtype):
    x = torch.randn(300, dtype=dtype, device="cuda")
    y = LogSumExpFwdOp(dtype=dtype, dim=-1)(x)
    atol, rtol = ref_tolerance(dtype)
    assert y.shape == () and abs(float(y) - float(_lse_ref(x, -1))) <= atol + rtol * abs(float(y))
    x3 = torch.randn(4, 128, 4096, dtype=dtype, device="cuda")
    y3 = LogSumExpFwdOp(dtype=dtype, dim=[0, 2])(x3)
    assert_close_np(to_np(y3), _lse_ref(x3, [0, 2]), atol, rtol, "lse multidim")


@pytest.mark.gpu
@pytest.mark.parametrize("rows", [64, 8192])  # 4 wavefronts per row / 1 per row
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_logsumexp_special_rows(rows, dtype):
    # Finite maxima beyond 2e38 (up to the dtype's largest finite value) must
    # stay finite, as torch.logsumexp keeps them: shift by the max unless it
    # is infinite.
    big = torch.finfo(dtype).max
    x = torch.randn(rows, 4096, device="cuda") * 2
    x[0] = float("-inf")
    x[1, 17] = float("inf")
    x[2, 4000] = float("nan")
    x[3] = 1e30
    x[4, :100] = float("-inf")
    x[5, 7] = 3e38
    x[6] = -3e38
    x[7] = big
    x[8] = -big
    x[9, :2048] = -3e38
    x[9, 2048:] = float("-inf")
    x[10, 5] = float("inf")
    x[10, 6] = float("-inf")
    x[10, 7] = 3e38
    x[11, 3000] = 3e38
    x[11, 3001] = float("nan")
    x = x.to(dtype)
    y = LogSumExpFwdOp(dtype=dtype)(x)
    ref = orc.logsumexp(to_np(x), NAMES[dtype])
    assert np.isfinite(ref[[3, 5, 6, 7, 8, 9]]).all()
    atol, rtol = ref_tolerance(dtype)
    assert_close_np(to_np(y), ref, atol, rtol, "lse special")


@pytest.mark.smoke
def test_logsumexp_eval_roofline_contract():
    with pytest.raises(RuntimeError, match="requires a prior"):
        LogSumExpFwdOp(dtype=torch.float16).eval_roofline()
    with pytest.raises(ValueError, match="Unsupported op_kind"):
        LogSumExpKernel(4, 4, "softmax", torch.float32)


@pytest.mark.gpu
def test_logsumexp_eval_roofline():
    M, N = 64, 256
    op = LogSumExpFwdOp(dim=-1, dtype=torch.float16)
    op(torch.randn(M, N, dtype=torch.float16, device="cuda"))
    assert op.eval_roofline() == (4 * M * N, (M * N + M) * 2)


# -- argmax -----------------------------------------------------------------------------
class ArgmaxTest(ArgmaxWorkload, TestBase):
    def __init__(self, m, n, dtype):
        super().__init__((m, n), dtype)

    def ref_program(self, x):
        return torch.from_numpy(orc.argreduce(to_np(x), -1)).to(x.device)


@pytest.mark.gpu
@pytest.mark.parametrize(
    "m, n, dtype",
    [
        pytest.param(128, 512, torch.float32, marks=pytest.mark.smoke),
        pytest.param(128, 512, torch.float16, marks=pytest.mark.smoke),
        pytest.param(128, 512, torch.bfloat16, marks=pytest.mark.smoke),
        pytest.param(256, 4096, torch.float16, marks=pytest.mark.full),
        pytest.param(256, 4096, torch.bfloat16, marks=pytest.mark.full),
        pytest.param(128, 300, torch.float16, marks=pytest.mark.full),
        pytest.param(128, 300, torch.bfloat16, marks=pytest.mark.full),
        pytest.param(129, 512, torch.float16, marks=pytest.mark.full),
        pytest.param(8192, 4096, torch.float32, marks=pytest.mark.full),
        pytest.param(4, 102400, torch.bfloat16, marks=pytest.mark.full),
    ],
)
def test_argmax_op(m, n, dtype):
    test = ArgmaxTest(m, n, dtype)
    test.check(ArgmaxFwdOp(dtype=dtype, dim=-1), *test.gen_inputs(), compare=_exact_compare)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_argmax_ties_nan_and_zeros(dtype):
    x = torch.randint(-3, 4, (512, 777), device="cuda").to(dtype)  # dense ties
    x[0] = float("-inf")
    x[1, [100, 700]] = float("nan")
    x[2] = 0.0
    x[2, :9] = -0.0
    x[3, 776] = float("inf")
    x[4] = float("nan")
    y = ArgmaxFwdOp(dtype=dtype, dim=-1)(x)
    np.testing.assert_array_equal(to_np(y), orc.argreduce(to_np(x), -1))
    np.testing.assert_array_equal(to_np(y), x.cpu().argmax(dim=-1).numpy())


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_argmax_non_contiguous(dtype):
    x = torch.randn(128, 1024, dtype=dtype, device="cuda")[:, :512]
    y = ArgmaxFwdOp(dtype=dtype, dim=-1)(x)
    assert torch.equal(y.cpu(), torch.from_numpy(orc.argreduce(to_np(x.contiguous()), -1)))


@pytest.mark.gpu
@pytest.mark.parametrize(
    "shape, dim, keepdim, dtype",
    [
        ((2, 64, 512), -1, False, torch.float16),
        ((2, 4, 8, 512), -1, False, torch.bfloat16),
        ((512,), -1, False, torch.float32),
        ((4, 8, 256), 0, False, torch.float16),
        ((4, 8, 256), 0, True, torch.float32),
        ((2, 4, 8, 256), 0, True, torch.bfloat16),
        ((128, 512), -1, True, torch.float16),
        ((512, 4, 32), 0, False, torch.float16),
        ((4, 32, 512), 1, False, torch.float16),
        ((4, 32, 512), -1, True, torch.bfloat16),
    ],
)
def test_argmax_dims(shape, dim, keepdim, dtype):
    x = torch.randn(*shape, dtype=dtype, device="cuda")
    y = ArgmaxFwdOp(dtype=dtype, dim=dim, keepdim=keepdim)(x)
    ref = x.cpu().argmax(dim=dim, keepdim=keepdim)
    assert y.shape == ref.shape and y.dtype == torch.int64
    assert torch.equal(y.cpu(), ref)


@pytest.mark.gpu
@pytest.mark.parametrize("shape, dtype", [((16, 64), torch.float16), ((16, 64), torch.bfloat16),
                                          ((16, 64), torch.float32), ((512,), torch.float16),
                                          ((4, 8, 32), torch.float16), ((2, 4, 8, 16), torch.float16),
                                          ((10, 30), torch.float16)])
def test_argmax_dim_none(shape, dtype):
    x = torch.randn(*shape, dtype=dtype, device="cuda")
    ref = torch.argmax(x.cpu())
    y = ArgmaxFwdOp(dtype=dtype, dim=None)(x)
    assert y.dtype == torch.int64 and y.shape == ref.shape and torch.equal(y.cpu(), ref)
    yk = ArgmaxFwdOp(dtype=dtype, dim=None, keepdim=True)(x)
    assert yk.shape == tuple(1 for _ in shape) and torch.equal(yk.reshape(()).cpu(), ref)


@pytest.mark.smoke
@pytest.mark.parametrize("dim", [[0, 1], (0, 1)])
def test_argmax_rejects_multidim(dim):
    with pytest.raises((TypeError, ValueError)):
        ArgmaxFwdOp(dtype=torch.float16, dim=dim)


@pytest.mark.smoke
def test_argreduce_kernel_contract():
    with pytest.raises(ValueError, match="Unsupported op_kind"):
        ArgreduceKernel(4, 4, "argsort", torch.float32)
    with pytest.raises(ValueError, match="empty"):
        ArgreduceKernel(4, 0, "argmax", torch.float32)
