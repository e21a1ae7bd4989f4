"""LerpFwdOp (scalar weight) and LerpTensorFwdOp (weight tensor) against the oracle.

Mirrors tests/ops/test_lerp_scalar.py and test_lerp_tensor.py of the
reference: same-shape inputs with the default and custom weights (0, 0.3,
0.5, 0.7, 1, -1.5, 2), the manifest broadcast shapes, NaN propagation, the
dtype rejections and messages, the roofline and the constructor-named
attributes.  The reference's golden is torch.lerp; the oracle restates it
(pinned against torch.lerp in tests/test_oracle_pins.py).  Half-precision
results must equal the oracle's bit for bit (one fp32 fma rounded once on
both sides); fp32 results within one ulp (the oracle emulates the fma in
fp64).  torch.lerp on the GPU is checked too, at the reference's tolerances.
"""

import numpy as np
import pytest
import torch

from oracle import tileops_oracle as orc
from tests._util import NAMES, assert_bits_equal, to_np
from tileops.benchmark.msprof import _extract_op_init_args
from tileops.kernels.elementwise.lerp_scalar import LerpScalarFwdKernel
from tileops.kernels.elementwise.lerp_tensor import LerpTensorFwdKernel
from tileops.ops.elementwise.lerp_scalar import LerpFwdOp
from tileops.ops.elementwise.lerp_tensor import LerpTensorFwdOp

DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def _tol(dtype):
    # tests/ops/test_lerp_scalar.py:33-38 of the reference
    if dtype == torch.float16:
        return {"atol": 1e-3, "rtol": 1e-3}
    if dtype == torch.bfloat16:
        return {"atol": 1e-2, "rtol": 1e-2}
    return {"atol": 1e-6, "rtol": 1e-6}


def _check(out, a, b, w, dtype, what):
    want = orc.lerp(to_np(a), to_np(b), w if np.isscalar(w) else to_np(w), NAMES[dtype])
    got = to_np(out)
    assert got.shape == want.shape, what
    if dtype == torch.float32:
        ng, nw = np.isnan(got), np.isnan(want)
        assert np.array_equal(ng, nw), f"{what}: NaN positions"
        gi = got[~ng].view(np.int32).astype(np.int64)
        wi = want[~nw].view(np.int32).astype(np.int64)
        assert np.abs(gi - wi).max(initial=0) <= 1, f"{what}: more than one ulp from the oracle"
    else:
        assert_bits_equal(got, want, what)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("weight", [0.0, 0.3, 0.5, 0.7, 1.0, -1.5, 2.0])
def test_lerp_scalar_weights(weight, dtype):
    shape = (64, 128)
    a = torch.randn(shape, device="cuda", dtype=dtype)
    b = torch.randn(shape, device="cuda", dtype=dtype)
    out = LerpFwdOp(input=shape, end=shape, dtype=dtype, weight=weight)(a, b)
    _check(out, a, b, weight, dtype, f"lerp w={weight} {dtype}")
    torch.testing.assert_close(out, torch.lerp(a, b, weight), **_tol(dtype))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
def test_lerp_scalar_default_weight(dtype):
    shape = (4, 8)
    a = torch.randn(shape, device="cuda", dtype=dtype)
    b = torch.randn(shape, device="cuda", dtype=dtype)
    op = LerpFwdOp(input=shape, end=shape, dtype=dtype)
    assert op.weight == 0.5
    _check(op(a, b), a, b, 0.5, dtype, f"lerp default {dtype}")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("a_shape, b_shape", [
    ((3, 1), (1, 4)),
    ((2, 512, 768), (1, 1, 768)),
    ((2, 512, 768), (2, 512, 1)),
    ((16, 256, 56, 56), (256, 1, 1)),
    ((1024, 4096), (1, 4096)),
    ((1024, 11008), (1024, 11008)),
    ((5, 1, 77), (3, 1)),
    ((9,), ()),
])
def test_lerp_scalar_broadcast(a_shape, b_shape, dtype):
    a = torch.randn(a_shape, device="cuda", dtype=dtype)
    b = torch.randn(b_shape, device="cuda", dtype=dtype)
    out = LerpFwdOp(input=a_shape, end=b_shape, dtype=dtype, weight=0.3)(a, b)
    assert tuple(out.shape) == tuple(torch.broadcast_shapes(a_shape, b_shape))
    _check(out, a, b, 0.3, dtype, f"lerp bcast {a_shape} {b_shape} {dtype}")


@pytest.mark.gpu
def test_lerp_scalar_nan_semantics():
    a = torch.randn(4096, device="cuda")
    b = torch.randn(4096, device="cuda")
    a[0::8] = float("nan")
    b[1::8] = float("nan")
    b[2::8] = float("inf")
    out = LerpFwdOp(input=(4096,), end=(4096,), dtype=torch.float32, weight=0.5)(a, b)
    _check(out, a, b, 0.5, torch.float32, "lerp nan")
    assert torch.equal(torch.isnan(out), torch.isnan(torch.lerp(a, b, 0.5)))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shapes", [
    ((1024, 1024), (1024, 1024), (1024, 1024)),
    ((4, 1, 64), (3, 1), (64,)),
    ((2, 512, 768), (1, 1, 768), (2, 512, 1)),
    ((33, 17), (33, 17), ()),
])
def test_lerp_tensor(shapes, dtype):
    sa, sb, sw = shapes
    a = torch.randn(sa, device="cuda", dtype=dtype)
    b = torch.randn(sb, device="cuda", dtype=dtype)
    w = (torch.rand(sw, device="cuda") * 3 - 1).to(dtype)  # both sides of |w| < 0.5
    out = LerpTensorFwdOp(input=sa, end=sb, weight=sw, dtype=dtype)(a, b, w)
    assert tuple(out.shape) == tuple(torch.broadcast_shapes(sa, sb, sw))
    _check(out, a, b, w, dtype, f"lerp_tensor {shapes} {dtype}")
    torch.testing.assert_close(out, torch.lerp(a, b, w), **_tol(dtype))


@pytest.mark.gpu
def test_lerp_storage_offset_operands():
    base = torch.randn(1 + 64 * 64, device="cuda", dtype=torch.bfloat16)
    a = base[1:].view(64, 64)
    b = torch.randn(64, 64, device="cuda", dtype=torch.bfloat16)
    w = torch.rand(64, 65, device="cuda").to(torch.bfloat16)[:, 1:]
    out = LerpTensorFwdOp(input=(64, 64), end=(64, 64), weight=(64, 64),
                          dtype=torch.bfloat16)(a, b, w)
    _check(out, a, b, w, torch.bfloat16, "lerp_tensor offset")
    out = LerpFwdOp(input=(64, 64), end=(64, 64), dtype=torch.bfloat16, weight=0.7)(b, a)
    _check(out, b, a, 0.7, torch.bfloat16, "lerp offset")


@pytest.mark.smoke
@pytest.mark.parametrize("bad", [torch.float8_e4m3fn, torch.int32])
def test_lerp_rejects_unsupported_dtype(bad):
    with pytest.raises(ValueError, match="LerpFwdOp does not support dtype"):
        LerpFwdOp(input=(4, 8), end=(4, 8), dtype=bad)
    with pytest.raises(ValueError, match="LerpTensorFwdOp does not support dtype"):
        LerpTensorFwdOp(input=(4,), end=(4,), weight=(4,), dtype=bad)
    with pytest.raises(ValueError, match="only supports dtypes"):
        LerpScalarFwdKernel(N_total=16, dtype=torch.int32, weight=0.5)
    with pytest.raises(ValueError, match="only supports dtypes"):
        LerpTensorFwdKernel(N_total=16, dtype=torch.int32)


@pytest.mark.gpu
def test_lerp_dtype_mismatch_rejected():
    op = LerpFwdOp(input=(4, 8), end=(4, 8), dtype=torch.float32)
    a = torch.randn(4, 8, device="cuda")
    with pytest.raises(ValueError, match="end.dtype"):
        op(a, a.half())
    opt = LerpTensorFwdOp(input=(4, 8), end=(4, 8), weight=(4, 8), dtype=torch.float32)
    with pytest.raises(ValueError, match="weight.dtype"):
        opt(a, a, a.half())


@pytest.mark.smoke
def test_lerp_eval_roofline_and_init_args():
    op = LerpFwdOp(input=(64, 128), end=(1, 128), dtype=torch.float16, weight=0.3)
    n = 64 * 128
    assert op.eval_roofline() == (3 * n, 4 * n * 2)
    assert _extract_op_init_args(op) == {"input": (64, 128), "end": (1, 128),
                                         "dtype": torch.float16, "weight": 0.3}
    opt = LerpTensorFwdOp(input=(8, 4), end=(8, 4), weight=(1, 4), dtype=torch.float32)
    assert opt.eval_roofline() == (96, 4 * 32 * 4)
    assert _extract_op_init_args(opt) == {"input": (8, 4), "end": (8, 4), "weight": (1, 4),
                                          "dtype": torch.float32}
