"""ClampMinFwdOp against the oracle.

Mirrors test_clamp_min.py of the reference (the min-only form of
test_clamp_scalar.py): the same sizes, dtypes, bounds, NaN / inf semantics,
``min=None`` rejection and roofline; the golden is the oracle's
``clamp_scalar(x, dtype, min, None)`` (torch.clamp_min(x.float(), min) cast
back), compared bit for bit since the kernel's result is a selected input or
the rounded bound.
"""

import numpy as np
import pytest
import torch

from oracle import tileops_oracle as orc
from tests._util import NAMES, assert_bits_equal, from_np, to_np
from tileops.kernels.elementwise.clamp_scalar import ClampScalarFwdKernel
from tileops.ops.elementwise.clamp_min import ClampMinFwdOp
from tileops.workloads.workload_base import FixtureBase

SIZES_DTYPES = [
    pytest.param(1_048_576, torch.float32, marks=[pytest.mark.smoke, pytest.mark.packaging]),
    pytest.param(1_048_576, torch.float16, marks=pytest.mark.smoke),
    pytest.param(1_048_576, torch.bfloat16, marks=pytest.mark.smoke),
    pytest.param(4_000_000, torch.float16, marks=pytest.mark.full),
    pytest.param(4_000_000, torch.bfloat16, marks=pytest.mark.full),
    # ragged: not a multiple of the 16-byte pack (scalar tail)
    pytest.param(1_000_003, torch.bfloat16, marks=pytest.mark.full),
]


class ClampMinFixture(FixtureBase):
    PARAMS = [("n_total, dtype", SIZES_DTYPES)]


def _golden(x: torch.Tensor, min_val: float) -> np.ndarray:
    return orc.clamp_scalar(to_np(x), NAMES[x.dtype], min_val, None)


@pytest.mark.gpu
@ClampMinFixture
def test_clamp_min_op(n_total, dtype):
    x = torch.randn(n_total, device="cuda").to(dtype)
    got = ClampMinFwdOp(N_total=n_total, dtype=dtype, min=-0.5)(x)
    assert got.shape == x.shape and got.dtype == dtype
    assert_bits_equal(to_np(got), _golden(x, -0.5), f"clamp_min {dtype}")


@pytest.mark.gpu
@pytest.mark.parametrize("min_val", [-0.5, 0.0, 0.25, float("nan"), float("-inf")])
def test_clamp_min_bounds(min_val):
    for dtype in (torch.float32, torch.float16, torch.bfloat16):
        x = torch.randn(1024, device="cuda").to(dtype)
        got = ClampMinFwdOp(N_total=1024, dtype=dtype, min=min_val)(x)
        assert_bits_equal(to_np(got), _golden(x, min_val), f"clamp_min {min_val} {dtype}")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_clamp_min_nan_inf_semantics(dtype):
    """NaN inputs stay NaN; +-inf and finite inputs follow torch.clamp_min."""
    n_total = 4096
    x = torch.randn(n_total, device="cuda").to(dtype)
    x[0::8] = float("nan")
    x[1::8] = float("inf")
    x[2::8] = float("-inf")
    got = ClampMinFwdOp(N_total=n_total, dtype=dtype, min=-0.5)(x)
    assert_bits_equal(to_np(got), _golden(x, -0.5), f"clamp_min specials {dtype}")
    assert torch.equal(torch.isnan(got), torch.isnan(x))


@pytest.mark.gpu
def test_clamp_min_keeps_shape():
    x = torch.randn(3, 77, 5, device="cuda", dtype=torch.float16)
    got = ClampMinFwdOp(N_total=x.numel(), dtype=torch.float16, min=0.0)(x)
    assert got.shape == x.shape
    assert_bits_equal(to_np(got), _golden(x, 0.0), "clamp_min 3-d")


def test_clamp_min_oracle_matches_torch():
    """The golden itself against torch.clamp_min on the CPU, NaN / inf included."""
    x = torch.randn(4096)
    x[0::8] = float("nan")
    x[1::8] = float("inf")
    x[2::8] = float("-inf")
    for dtype in (torch.float32, torch.float16, torch.bfloat16):
        xd = x.to(dtype)
        for lo in (-0.5, 0.0, float("nan")):
            want = torch.clamp_min(xd.float(), lo).to(dtype)
            got = from_np(_golden(xd, lo), want, dtype)
            assert torch.equal(torch.isnan(got), torch.isnan(want))
            ok = ~torch.isnan(want)
            assert torch.equal(got[ok], want[ok]), (dtype, lo)


@pytest.mark.smoke
def test_clamp_min_none_rejected():
    with pytest.raises(ValueError, match=r"requires min"):
        ClampMinFwdOp(N_total=16, dtype=torch.float32, min=None)


@pytest.mark.smoke
def test_clamp_min_rejects_non_float_dtype():
    with pytest.raises(ValueError, match="only supports dtypes"):
        ClampScalarFwdKernel(N_total=16, dtype=torch.int32, min_val=-0.5)


@pytest.mark.smoke
def test_clamp_min_uses_the_clamp_kernel_without_upper_bound():
    op = ClampMinFwdOp(N_total=16, dtype=torch.float16, min=-0.5)
    assert isinstance(op.kernel, ClampScalarFwdKernel)
    assert op.max is None and op.min == -0.5


@pytest.mark.smoke
def test_clamp_min_eval_roofline():
    N = 1_048_576
    op = ClampMinFwdOp(N_total=N, dtype=torch.float16, min=-0.5)
    assert op.eval_roofline() == (N, 2 * N * 2)
