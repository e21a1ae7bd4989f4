"""GatedDeltaNetDecodeFwdOp against the oracle.

The reference has no GDN decode op or test; the golden is the oracle's
gdn_decode, one token of the restated golden_gdn_sequential
(examples/gdn_prefill/probe/gdn_prefill_probe.py:60-77), pinned in
tests/test_oracle_pins.py against the token loop and closed forms.  Inputs
are exact in their storage dtypes; the kernel computes in fp32, the oracle in
fp64.  Tolerances: the fp32 state at rtol = atol = 2e-5 (fp32 rounding of
K-term sums); o at one unit in the last place of its dtype (rtol 8e-3 bf16,
1e-3 fp16, 2e-5 fp32), since both sides round once to it.  Shapes cover both
row-slice widths the kernel picks (16 packs of 4 columns where they divide
the value width, else 8), K = 32 .. 256 (1 to 16 rows per thread), value
widths from one 32-column block to the 4096 maximum, several batches and
heads, a custom scale, the serving shape, and a state over 128 MiB (read
with non-temporal loads); a chained test runs a prefill and continues it
with decode steps, and the C-ABI's in-place form must equal the
out-of-place one bit for bit.
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle import tileops_oracle as orc
from tests._util import NAMES, assert_close_np, to_np
from tileops import _native
from tileops.kernels.linear_attention.gdn_decode import GDNDecodeKernel
from tileops.ops.linear_attention import GatedDeltaNetDecodeFwdOp, GatedDeltaNetPrefillFwdOp
from tileops.workloads.linear_attention import GdnDecodeWorkload, GdnPrefillWorkload

_F16, _BF16, _F32 = torch.float16, torch.bfloat16, torch.float32
STATE_TOL = 2e-5
O_RTOL = {_BF16: 8e-3, _F16: 1e-3, _F32: 2e-5}
O_ATOL = 2e-5

# (B, H, K, V, dtype, scale, id)
_CASES = [
    (1, 32, 128, 128, _BF16, None, "serving-b1-h32"),
    (8, 32, 128, 128, _BF16, None, "serving-b8-h32"),
    (32, 16, 128, 128, _BF16, None, "batch32-h16"),
    (2, 4, 64, 64, _F16, None, "k64-fp16"),
    (1, 2, 32, 32, _F32, None, "k32-one-block-fp32"),
    (1, 4, 96, 160, _F16, 0.25, "k96-v160-custom-scale"),
    (2, 3, 256, 64, _BF16, None, "k256"),
    (1, 2, 160, 1024, _F32, None, "k160-v1024"),
    (3, 5, 224, 96, _BF16, None, "k224-v96"),
    (2, 2, 192, 4096, _BF16, None, "k192-v4096-max"),
    (1, 4, 96, 384, _F32, None, "k96-v384"),
    (2, 2, 32, 64, _F32, None, "k32-v64"),
    (1, 3, 224, 128, _F16, None, "k224-v128"),
    (66, 32, 128, 128, _BF16, None, "state-over-128MiB-nontemporal-loads"),
]


def _check_step(q, k, v, g, beta, state, o, ns, scale, dtype, label):
    ref_o, ref_s = orc.gdn_decode(to_np(q), to_np(k), to_np(v), to_np(g), to_np(beta),
                                  to_np(state), scale, NAMES[dtype])
    err_s = float(np.max(np.abs(to_np(ns) - ref_s) / (STATE_TOL + STATE_TOL * np.abs(ref_s))))
    print(f"[gdn decode {label}] largest state error / bound {err_s:.3f}")
    assert_close_np(to_np(ns), ref_s, STATE_TOL, STATE_TOL, f"new_state {label}")
    assert_close_np(to_np(o), ref_o, O_ATOL, O_RTOL[dtype], f"o {label}")


@pytest.mark.gpu
@pytest.mark.parametrize("B, H, K, V, dtype, scale, case_id",
                         [pytest.param(*c, id=c[-1]) for c in _CASES])
def test_gdn_decode(B, H, K, V, dtype, scale, case_id):
    torch.manual_seed(hash(case_id) % 1000)
    q, k, v, g, beta, state = GdnDecodeWorkload(B, H, K, V, dtype).gen_inputs()
    op = GatedDeltaNetDecodeFwdOp(B, H, K, V, dtype=dtype, scale=scale)
    o, ns = op(q, k, v, g, beta, state)
    assert o.shape == (B, H, V) and o.dtype == dtype
    assert ns.shape == (B, H, K, V) and ns.dtype == _F32
    _check_step(q, k, v, g, beta, state, o, ns, op.scale, dtype, case_id)


@pytest.mark.gpu
def test_gdn_decode_continues_a_prefill():
    # a prefill over T tokens, then n decode steps from its final state, equal
    # the recurrence over all T + n tokens
    B, T, H, n = 2, 200, 3, 4
    torch.manual_seed(5)
    q, k, v, g, beta = GdnPrefillWorkload(B, T + n, H, 128, 128).gen_inputs()
    h0 = torch.randn(B, H, 128, 128, device=q.device)
    pre = GatedDeltaNetPrefillFwdOp(B, T, H)
    o_pre, state = pre(q[:, :T], k[:, :T], v[:, :T], g[:, :T], beta[:, :T], h0)
    dec = GatedDeltaNetDecodeFwdOp(B, H)
    outs = []
    for t in range(T, T + n):
        step = (q[:, t], k[:, t], v[:, t], g[:, t], beta[:, t])
        o_t, ns = dec(*step, state)
        _check_step(*step, state, o_t, ns, dec.scale, _BF16, f"token {t}")
        outs.append(o_t)
        state = ns
    o_ref, s_ref = orc.gdn_sequential(*(to_np(t) for t in (q, k, v, g, beta)), to_np(h0),
                                      pre.scale)
    o_ref = orc.round_to("bfloat16", o_ref)
    assert_close_np(to_np(torch.stack(outs, 1)), o_ref[:, T:], 1e-2, 1e-2, "decoded o")
    assert_close_np(to_np(o_pre), o_ref[:, :T], 1e-2, 1e-2, "prefill o")
    assert_close_np(to_np(state), s_ref, 1e-2, 1e-2, "state after prefill + decode")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [_BF16, _F32])
def test_gdn_decode_in_place_equals_out_of_place(dtype):
    B, H, K, V = 4, 8, 128, 256
    torch.manual_seed(6)
    q, k, v, g, beta, state = GdnDecodeWorkload(B, H, K, V, dtype).gen_inputs()
    before = state.clone()
    o, ns = GatedDeltaNetDecodeFwdOp(B, H, K, V, dtype=dtype)(q, k, v, g, beta, state)
    assert torch.equal(state, before)  # the Op returns the state functionally
    o2 = torch.empty_like(o)
    lib = _native.lib()
    code = lib.tileops_gdn_decode_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(),
        state.data_ptr(), o2.data_ptr(), state.data_ptr(), B, H, K, V,
        ctypes.c_float(K**-0.5), _native.dtype_code(dtype), _native.stream_of(q))
    _native.check(code, "tileops_gdn_decode_fwd")
    torch.cuda.synchronize()
    assert torch.equal(state, ns) and torch.equal(o2, o)


@pytest.mark.gpu
def test_gdn_decode_misaligned_state_view():
    # a contiguous state view 4 bytes past a 16-byte boundary is realigned
    B, H, K, V = 1, 2, 32, 64
    torch.manual_seed(8)
    q, k, v, g, beta, state = GdnDecodeWorkload(B, H, K, V, _F32).gen_inputs()
    flat = torch.empty(state.numel() + 1, device=state.device)
    shifted = flat[1:].view(B, H, K, V)
    shifted.copy_(state)
    assert shifted.data_ptr() % 16 == 4
    op = GatedDeltaNetDecodeFwdOp(B, H, K, V, dtype=_F32)
    o, ns = op(q, k, v, g, beta, shifted)
    o_ref, ns_ref = op(q, k, v, g, beta, state)
    assert torch.equal(o, o_ref) and torch.equal(ns, ns_ref)


@pytest.mark.smoke
def test_gdn_decode_default_scale_and_roofline():
    op = GatedDeltaNetDecodeFwdOp(2, 4, 128, 64, dtype=_F16)
    assert op.kernel.scale == pytest.approx(128**-0.5)
    assert GatedDeltaNetDecodeFwdOp(2, 4, dtype=_F16, scale=0.5).kernel.scale == 0.5
    flops, nbytes = op.eval_roofline()
    assert flops == 8 * (7 * 128 * 64 + 2 * 128 + 7 * 64)
    assert nbytes == 8 * (8 * 128 * 64 + (2 * 128 + 2 * 64) * 2 + 8)


@pytest.mark.smoke
def test_gdn_decode_kernel_contract():
    with pytest.raises(ValueError, match="only supports dtypes"):
        GDNDecodeKernel(1, 2, 64, 64, torch.int32)
    for K, V in ((48, 64), (288, 64), (64, 80), (64, 8192), (0, 64)):
        with pytest.raises(ValueError, match="multiple of 32"):
            GDNDecodeKernel(1, 2, K, V, _BF16)
    with pytest.raises(ValueError, match="batch > 0"):
        GDNDecodeKernel(0, 2, 64, 64, _BF16)
    with pytest.raises(ValueError, match="unknown config"):
        GDNDecodeKernel(1, 2, 64, 64, _BF16, config={"tile": 3})


@pytest.mark.smoke
def test_gdn_decode_needs_device_tensors():
    # the product path has no host fallback
    op = GatedDeltaNetDecodeFwdOp(1, 2, 32, 32, dtype=_F32)
    q = torch.zeros(1, 2, 32)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        op(q, q, q, torch.zeros(1, 2), torch.zeros(1, 2), torch.zeros(1, 2, 32, 32))
