"""tileops_gdn_prefill_fwd_noalloc -- the entry point that allocates nothing --
against tileops_gdn_prefill_fwd, both called through the C ABI.

The two entry points run the same kernels; the allocation-free one keeps the
chunk records in the library's fixed device array and so works through long
sequences in segments, carrying the state between them.  Its results must
equal the workspace entry point's bit for bit: on two calls in a row (the
second with a smaller input), the first long enough to take several
segments and starting from a given state.  A call whose heads cannot fit
the array is rejected before any launch.
"""

import pytest
import torch

from tileops import _native
from tileops.workloads.linear_attention import GdnPrefillWorkload

BF16 = _native.DTYPE_CODES[torch.bfloat16]
SCRATCH_BYTES = 16 << 20
RECORD_BYTES = 17408


def _args(q, k, v, g, beta, h0, o, hT, B, T, H):
    return (q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(),
            h0.data_ptr() if h0 is not None else None, o.data_ptr(), hT.data_ptr(),
            B, T, H, 128, 128, 64, 128**-0.5, BF16)


def _run_both(B, T, H, with_h0):
    lib = _native.lib()
    q, k, v, g, beta = GdnPrefillWorkload(B, T, H, 128, 128).gen_inputs()
    h0 = torch.randn(B, H, 128, 128, device="cuda") * 0.1 if with_h0 else None
    stream = _native.stream_of(q)
    o_ref = torch.empty_like(v)
    hT_ref = torch.empty(B, H, 128, 128, device="cuda")
    need = lib.tileops_gdn_prefill_workspace_bytes(B, T, H, 128, 128, 64)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    code = lib.tileops_gdn_prefill_fwd(*_args(q, k, v, g, beta, h0, o_ref, hT_ref, B, T, H),
                                       ws.data_ptr(), ws.numel(), stream)
    _native.check(code, "tileops_gdn_prefill_fwd")
    o = torch.full_like(v, float("nan"))
    hT = torch.full((B, H, 128, 128), float("nan"), device="cuda")
    code = lib.tileops_gdn_prefill_fwd_noalloc(*_args(q, k, v, g, beta, h0, o, hT, B, T, H),
                                               stream)
    _native.check(code, "tileops_gdn_prefill_fwd_noalloc")
    torch.cuda.synchronize()
    return o, hT, o_ref, hT_ref


@pytest.mark.gpu
def test_noalloc_matches_the_workspace_entry_point_on_two_calls():
    # first call: 32 heads need 544 KiB per chunk, so the 16 MiB array holds
    # 30 chunks and T = 2048 (32 chunks) runs as two segments
    B, T, H = 2, 2048, 16
    assert (SCRATCH_BYTES // (B * H * RECORD_BYTES)) < (T + 63) // 64
    o, hT, o_ref, hT_ref = _run_both(B, T, H, with_h0=True)
    assert torch.equal(o, o_ref), "o differs (long call)"
    assert torch.equal(hT, hT_ref), "final state differs (long call)"
    # second call, smaller and ragged, from a zero state
    o, hT, o_ref, hT_ref = _run_both(1, 300, 4, with_h0=False)
    assert torch.equal(o, o_ref), "o differs (second call)"
    assert torch.equal(hT, hT_ref), "final state differs (second call)"


@pytest.mark.gpu
def test_noalloc_rejects_heads_beyond_the_array():
    lib = _native.lib()
    H = SCRATCH_BYTES // RECORD_BYTES + 1  # one record per head no longer fits
    fake = 256  # aligned, never dereferenced: the call returns before any launch
    code = lib.tileops_gdn_prefill_fwd_noalloc(fake, fake, fake, fake, fake, None, fake, fake,
                                               1, 64, H, 128, 128, 64, 0.1, BF16, None)
    assert code == -4  # TILEOPS_EWORKSPACE


@pytest.mark.gpu
def test_noalloc_zero_length_passes_the_state_through_for_any_head_count():
    # with T = 0 there are no chunks and no scratch is used, so the head
    # count that the array bounds for T > 0 must not be rejected
    lib = _native.lib()
    B, H = 1, SCRATCH_BYTES // RECORD_BYTES + 1
    h0 = torch.randn(B, H, 128, 128, device="cuda")
    hT = torch.full_like(h0, float("nan"))
    e = torch.empty(B, 0, H, 128, device="cuda", dtype=torch.bfloat16)
    z = torch.empty(B, 0, H, device="cuda")
    code = lib.tileops_gdn_prefill_fwd_noalloc(*_args(e, e, e, z, z, h0, e, hT, B, 0, H),
                                               _native.stream_of(h0))
    _native.check(code, "tileops_gdn_prefill_fwd_noalloc")
    torch.cuda.synchronize()
    assert torch.equal(hT, h0)
