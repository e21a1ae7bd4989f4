"""AddFwdOp / SubFwdOp against the oracle.

Mirrors test_add.py / test_sub.py of the reference: the manifest shapes
(same-shape and broadcast: a per-channel [C, 1, 1] operand, a [1, N] bias),
the float dtypes and their tolerances, alpha other than 1, the dtype
rejection and the roofline.  The oracle is numpy broadcasting with fp32
opmath (pinned against torch.add / torch.sub in tests/test_oracle_pins.py);
the kernel reads broadcast operands through zero strides, so no copy is
made.
"""

import pytest
import torch

from oracle import tileops_oracle as orc
from tests._util import NAMES, assert_close_np, ref_tolerance, to_np
from tileops.ops.elementwise.add import AddFwdOp
from tileops.ops.elementwise.sub import SubFwdOp

SHAPES = [
    ((2048, 4096), (2048, 4096)),
    ((16, 256, 56, 56), (256, 1, 1)),
    ((1024, 4096), (1, 4096)),
    ((3, 1, 77), (5, 1)),        # both operands broadcast, ragged
    ((7,), ()),                  # scalar operand
    ((64,), ()),                 # scalar operand, whole packs
    ((1, 64), (32, 64)),         # the first operand broadcast
    ((4, 8, 1, 32), (8, 32, 1)),  # rows of one operand, columns of the other
]


@pytest.mark.gpu
@pytest.mark.parametrize("op_cls, sign", [(AddFwdOp, 1.0), (SubFwdOp, -1.0)])
@pytest.mark.parametrize("shapes", SHAPES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("alpha", [1, 0.5])
def test_add_sub(op_cls, sign, shapes, dtype, alpha):
    sa, sb = shapes
    a = torch.randn(sa, device="cuda").to(dtype)
    b = torch.randn(sb, device="cuda").to(dtype)
    op = op_cls(input=sa, other=sb, dtype=dtype, alpha=alpha)
    y = op(a, b)
    assert tuple(y.shape) == tuple(torch.broadcast_shapes(sa, sb)) and y.dtype == dtype
    want = orc.add(to_np(a), to_np(b), sign * alpha, NAMES[dtype])
    atol, rtol = ref_tolerance(dtype)
    assert_close_np(to_np(y), want, atol, rtol, f"{op_cls.__name__} {sa} {sb} {dtype} {alpha}")


@pytest.mark.gpu
def test_add_non_contiguous_operand():
    a = torch.randn(64, 128, device="cuda").t()  # strided view
    b = torch.randn(128, 1, device="cuda")
    y = AddFwdOp(input=(128, 64), other=(128, 1), dtype=torch.float32, alpha=2)(a, b)
    assert_close_np(to_np(y), orc.add(to_np(a), to_np(b), 2, "float32"), 1e-6, 1e-6, "strided")


@pytest.mark.smoke
def test_add_rejects_non_float_dtype():
    with pytest.raises(ValueError, match="does not support dtype"):
        AddFwdOp(input=(4,), other=(4,), dtype=torch.int32)


@pytest.mark.smoke
def test_add_sub_eval_roofline():
    op = AddFwdOp(input=(16, 256, 56, 56), other=(256, 1, 1), dtype=torch.float16)
    n = 16 * 256 * 56 * 56
    assert op.eval_roofline() == (n, 3 * n * 2)
    assert SubFwdOp(input=(8,), other=(8,), dtype=torch.float32, alpha=2).eval_roofline() == (16, 96)


@pytest.mark.gpu
@pytest.mark.parametrize("op_cls, sign", [(AddFwdOp, 1.0), (SubFwdOp, -1.0)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_add_sub_storage_offset_operands(op_cls, sign, dtype):
    # views that start one element into their storage are not 16-byte
    # aligned: the kernels must take their element-wise paths for them
    base = torch.randn(1 + 96 * 64, device="cuda").to(dtype)
    a = base[1:].view(96, 64)                       # same shape, misaligned
    b = torch.randn(96, 65, device="cuda").to(dtype)[:, 1:]  # row offset 1
    for other, oshape in ((b, (96, 64)), (b[:1], (1, 64)), (b[:, :1], (96, 1))):
        op = op_cls(input=(96, 64), other=oshape, dtype=dtype, alpha=0.5)
        y = op(a, other)
        want = orc.add(to_np(a), to_np(other), sign * 0.5, NAMES[dtype])
        atol, rtol = ref_tolerance(dtype)
        assert_close_np(to_np(y), want, atol, rtol, f"offset {op_cls.__name__} {oshape} {dtype}")
    # the second operand misaligned against an aligned first one, flat
    y = op_cls(input=(96 * 64,), other=(96 * 64,), dtype=dtype)(
        torch.randn(96 * 64, device="cuda").to(dtype), base[1:])
    assert y.shape == (96 * 64,)
