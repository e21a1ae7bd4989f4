"""MishFwdOp against the oracle.

Mirrors test_mish.py of the reference (the same sizes, dtypes, per-dtype
tolerances, dtype rejection and roofline); the golden is the oracle's
F.mish(x.float()).to(dtype), pinned against torch's F.mish in
tests/test_oracle_pins.py.  Adds the special values (NaN, +-inf, large
magnitudes where softplus saturates) and the in-place flag.
"""

import numpy as np
import pytest
import torch

from oracle import tileops_oracle as orc
from tests._util import NAMES, assert_close_np, from_np, ref_tolerance, to_np
from tileops.kernels.elementwise.mish import MishFwdKernel
from tileops.ops.elementwise.mish import MishFwdOp
from tileops.workloads.workload_base import FixtureBase

SIZES_DTYPES = [
    pytest.param(1_048_576, torch.float32, marks=[pytest.mark.smoke, pytest.mark.packaging]),
    pytest.param(1_048_576, torch.float16, marks=pytest.mark.smoke),
    pytest.param(1_048_576, torch.bfloat16, marks=pytest.mark.smoke),
    pytest.param(4_000_000, torch.float16, marks=pytest.mark.full),
    pytest.param(4_000_000, torch.bfloat16, marks=pytest.mark.full),
    pytest.param(1_000_003, torch.float32, marks=pytest.mark.full),  # scalar tail
]


class MishFixture(FixtureBase):
    PARAMS = [("n_total, dtype", SIZES_DTYPES)]


@pytest.mark.gpu
@MishFixture
def test_mish_op(n_total, dtype):
    x = (torch.randn(n_total, device="cuda") * 3).to(dtype)
    got = MishFwdOp(N_total=n_total, dtype=dtype)(x)
    atol, rtol = ref_tolerance(dtype)
    assert_close_np(to_np(got), orc.mish(to_np(x), NAMES[dtype]), atol, rtol, f"mish {dtype}")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_mish_special_values(dtype):
    vals = np.array([0.0, -0.0, 1.0, -1.0, 20.0, -20.0, 60.0, -60.0, 100.0, -100.0, 1e-3,
                     -1e-3, np.nan, np.inf, -np.inf], np.float32)
    x = from_np(orc.round_to(NAMES[dtype], vals), torch.empty(0, device="cuda"), dtype)
    got, want = to_np(MishFwdOp(N_total=x.numel(), dtype=dtype)(x)), orc.mish(to_np(x), NAMES[dtype])
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    atol, rtol = ref_tolerance(dtype)
    assert_close_np(got[ok], want[ok], atol, rtol, f"mish specials {dtype}")


@pytest.mark.gpu
def test_mish_inplace():
    x = torch.randn(3, 1000, device="cuda", dtype=torch.float16)
    want = orc.mish(to_np(x), "float16")
    out = MishFwdOp(N_total=x.numel(), dtype=torch.float16, inplace=True)(x)
    assert out.data_ptr() == x.data_ptr()
    assert_close_np(to_np(x), want, 1e-3, 1e-3, "mish in place")


@pytest.mark.smoke
def test_mish_rejects_non_float_dtype():
    with pytest.raises(ValueError, match="only supports dtypes"):
        MishFwdKernel(N_total=16, dtype=torch.int32)


@pytest.mark.smoke
def test_mish_eval_roofline():
    N = 1_048_576
    flops, nbytes = MishFwdOp(N_total=N, dtype=torch.float16).eval_roofline()
    assert flops == 4 * N and nbytes == 2 * N * 2
