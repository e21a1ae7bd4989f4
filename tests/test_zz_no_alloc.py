"""tileops_gdn_prefill_fwd_noalloc -- the entry point that allocates nothing --
against tileops_gdn_prefill_fwd, both called through the C ABI.

The two entry points run the same kernels; the allocation-free one keeps the
segment maps in the library's fixed device array.  Its results must equal
the workspace entry point's bit for bit (same segment plan): on two calls in
a row (the second with a smaller input), the first long enough to take
several segments and starting from a given state; on two calls issued on two
different streams one right after the other (the library orders them, since
both use the array); and for a head count so large that the sequence runs
as one segment, which needs no array.
"""

import pytest
import torch

from tileops import _native
from tileops.workloads.linear_attention import GdnPrefillWorkload

BF16 = _native.DTYPE_CODES[torch.bfloat16]


def _args(q, k, v, g, beta, h0, o, hT, B, T, H):
    return (q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(),
            h0.data_ptr() if h0 is not None else None, o.data_ptr(), hT.data_ptr(),
            B, T, H, 128, 128, 64, 128**-0.5, BF16)


def _inputs(B, T, H, with_h0):
    q, k, v, g, beta = GdnPrefillWorkload(B, T, H, 128, 128).gen_inputs()
    g = g * 0.01  # slow decay: the segment maps carry the state
    h0 = torch.randn(B, H, 128, 128, device="cuda") * 0.1 if with_h0 else None
    return q, k, v, g, beta, h0


def _reference(lib, inp, B, T, H, stream):
    q, k, v, g, beta, h0 = inp
    o = torch.empty_like(v)
    hT = torch.empty(B, H, 128, 128, device="cuda")
    need = lib.tileops_gdn_prefill_workspace_bytes(B, T, H, 128, 128, 64)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    code = lib.tileops_gdn_prefill_fwd(*_args(q, k, v, g, beta, h0, o, hT, B, T, H),
                                       ws.data_ptr(), ws.numel(), stream)
    _native.check(code, "tileops_gdn_prefill_fwd")
    return o, hT, need


def _noalloc(lib, inp, B, T, H, stream):
    q, k, v, g, beta, h0 = inp
    o = torch.full_like(v, float("nan"))
    hT = torch.full((B, H, 128, 128), float("nan"), device="cuda")
    torch.cuda.synchronize()  # the fills (current stream) are done before `stream` runs
    code = lib.tileops_gdn_prefill_fwd_noalloc(*_args(q, k, v, g, beta, h0, o, hT, B, T, H),
                                               stream)
    _native.check(code, "tileops_gdn_prefill_fwd_noalloc")
    return o, hT


@pytest.mark.gpu
def test_noalloc_matches_the_workspace_entry_point_on_two_calls():
    lib = _native.lib()
    stream = _native.stream_of(torch.empty(1, device="cuda"))
    # first call: 32 heads, 32 chunks -> eight segments, 13 maps per head
    B, T, H = 2, 2048, 16
    inp = _inputs(B, T, H, with_h0=True)
    o_ref, hT_ref, need = _reference(lib, inp, B, T, H, stream)
    assert need > 0  # the plan uses segment maps
    o, hT = _noalloc(lib, inp, B, T, H, stream)
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref), "o differs (long call)"
    assert torch.equal(hT, hT_ref), "final state differs (long call)"
    # second call, smaller and ragged, from a zero state
    inp = _inputs(1, 1300, 4, with_h0=False)
    o_ref, hT_ref, _ = _reference(lib, inp, 1, 1300, 4, stream)
    o, hT = _noalloc(lib, inp, 1, 1300, 4, stream)
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref), "o differs (second call)"
    assert torch.equal(hT, hT_ref), "final state differs (second call)"


@pytest.mark.gpu
def test_noalloc_calls_on_two_streams_do_not_race():
    lib = _native.lib()
    B, T, H = 2, 2048, 16
    inp1 = _inputs(B, T, H, with_h0=True)
    inp2 = _inputs(B, T, H, with_h0=False)
    s0 = _native.stream_of(torch.empty(1, device="cuda"))
    r1 = _reference(lib, inp1, B, T, H, s0)
    r2 = _reference(lib, inp2, B, T, H, s0)
    torch.cuda.synchronize()
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()  # default priority
    o1, hT1 = _noalloc(lib, inp1, B, T, H, sa.cuda_stream)
    o2, hT2 = _noalloc(lib, inp2, B, T, H, sb.cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(o1, r1[0]) and torch.equal(hT1, r1[1]), "first stream's call"
    assert torch.equal(o2, r2[0]) and torch.equal(hT2, r2[1]), "second stream's call"


@pytest.mark.gpu
def test_noalloc_runs_many_heads_as_one_segment():
    # 2000 heads fill the device without splitting the sequence: no maps,
    # no array
    lib = _native.lib()
    B, T, H = 1, 200, 2000
    assert lib.tileops_gdn_prefill_workspace_bytes(B, T, H, 128, 128, 64) == 0
    inp = _inputs(B, T, H, with_h0=False)
    stream = _native.stream_of(inp[0])
    o_ref, hT_ref, _ = _reference(lib, inp, B, T, H, stream)
    o, hT = _noalloc(lib, inp, B, T, H, stream)
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref) and torch.equal(hT, hT_ref)


@pytest.mark.gpu
def test_noalloc_zero_length_passes_the_state_through_for_any_head_count():
    lib = _native.lib()
    B, H = 1, 1000
    h0 = torch.randn(B, H, 128, 128, device="cuda")
    hT = torch.full_like(h0, float("nan"))
    e = torch.empty(B, 0, H, 128, device="cuda", dtype=torch.bfloat16)
    z = torch.empty(B, 0, H, device="cuda")
    code = lib.tileops_gdn_prefill_fwd_noalloc(*_args(e, e, e, z, z, h0, e, hT, B, 0, H),
                                               _native.stream_of(h0))
    _native.check(code, "tileops_gdn_prefill_fwd_noalloc")
    torch.cuda.synchronize()
    assert torch.equal(hT, h0)
