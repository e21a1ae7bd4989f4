"""BitwiseNotFwdOp against the oracle (torch.bitwise_not), bit for bit.

Mirrors test_bitwise_not.py of the reference: every admitted dtype (bool,
uint8, int8, int16, int32, int64) on the manifest sizes, the dtype rejection
and the roofline; adds ragged sizes (byte tail), extreme values and shapes.
"""

import numpy as np
import pytest
import torch

from oracle import tileops_oracle as orc
from tileops.kernels.elementwise.bitwise_not import BitwiseNotFwdKernel
from tileops.ops.elementwise.bitwise_not import BitwiseNotFwdOp
from tileops.workloads.elementwise import BitwiseNotWorkload

DTYPES = [torch.bool, torch.uint8, torch.int8, torch.int16, torch.int32, torch.int64]


@pytest.mark.gpu
@pytest.mark.parametrize("n_total", [1_048_576, 1_000_003, 13, 1])
@pytest.mark.parametrize("dtype", DTYPES)
def test_bitwise_not_op(n_total, dtype):
    (x,) = BitwiseNotWorkload((n_total,), dtype).gen_inputs()
    got = BitwiseNotFwdOp(N_total=n_total, dtype=dtype)(x)
    assert got.dtype == dtype and got.shape == x.shape
    np.testing.assert_array_equal(got.cpu().numpy(), orc.bitwise_not(x.cpu().numpy()))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES[1:])
def test_bitwise_not_extremes_and_shape(dtype):
    info = torch.iinfo(dtype)
    vals = torch.tensor([0, 1, -1 if info.min < 0 else 2, info.min, info.max, info.max - 1],
                        dtype=dtype)
    x = vals.repeat(7 * 5).reshape(7, 5, 6).cuda()
    got = BitwiseNotFwdOp(N_total=x.numel(), dtype=dtype)(x)
    assert got.shape == x.shape
    assert torch.equal(got.cpu(), torch.bitwise_not(x.cpu()))


def test_bitwise_not_oracle_matches_torch():
    rng = np.random.default_rng(3)
    for dtype in DTYPES:
        if dtype == torch.bool:
            x = torch.from_numpy(rng.integers(0, 2, 1000).astype(bool))
        else:
            x = torch.from_numpy(rng.integers(0, 256, 1000 * torch.empty(0, dtype=dtype)
                                              .element_size(), dtype=np.uint8)).view(dtype)
        np.testing.assert_array_equal(orc.bitwise_not(x.numpy()), torch.bitwise_not(x).numpy())


@pytest.mark.smoke
def test_bitwise_not_rejects_float_dtype():
    with pytest.raises(ValueError, match="does not support dtype"):
        BitwiseNotFwdOp(N_total=16, dtype=torch.float32)
    with pytest.raises(ValueError, match="only supports dtypes"):
        BitwiseNotFwdKernel(N_total=16, dtype=torch.float16)


@pytest.mark.smoke
def test_bitwise_not_eval_roofline():
    N = 1_048_576
    for dtype in DTYPES:
        flops, nbytes = BitwiseNotFwdOp(N_total=N, dtype=dtype).eval_roofline()
        assert flops == N and nbytes == 2 * N * dtype.itemsize
