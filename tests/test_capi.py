"""The C-ABI library: loads, exports every symbol include/tileops_hip.h declares,
and rejects bad arguments on the host before touching a GPU.  No kernel is
launched here (these run on hosts without a GPU)."""

import ctypes
import re
from pathlib import Path

import pytest

from tileops import _native

HEADER = Path(__file__).resolve().parents[1] / "include" / "tileops_hip.h"


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tileops_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not _native.LIB_PATH.is_file():
        pytest.fail(f"{_native.LIB_PATH} is not built (run __graft_entry__.build())")
    return _native.lib()


def test_header_declares_the_expected_entry_points():
    names = _declared_functions()
    for required in ("tileops_unary_fwd", "tileops_isfp_fwd", "tileops_gated_gelu_fwd",
                     "tileops_fused_add_layernorm_fwd", "tileops_logsumexp_fwd",
                     "tileops_argreduce_fwd", "tileops_mha_fwd", "tileops_gdn_prefill_fwd",
                     "tileops_gla_decode_fwd", "tileops_gdn_decode_fwd",
                     "tileops_bitwise_not_fwd"):
        assert required in names


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in _declared_functions() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_binding_table_covers_the_header():
    assert set(_native.SIGNATURES) == set(_declared_functions())


def test_version_and_error_strings(lib):
    assert lib.tileops_version() >= 100
    assert lib.tileops_error_string(0) == b"success"
    for code in (-1, -2, -3, -4):
        assert lib.tileops_error_string(code).startswith(b"tileops:")


def test_host_side_argument_rejection(lib):
    # every case returns before any HIP call
    assert lib.tileops_unary_fwd(0, None, None, 16, 7, 0.0, 0.0, 0, None) == -1  # dtype
    assert lib.tileops_unary_fwd(9, None, None, 16, 0, 0.0, 0.0, 0, None) == -1  # op
    assert lib.tileops_unary_fwd(2, None, None, 16, 0, 0.0, 0.0, 0, None) == -1  # clamp w/o bound
    assert lib.tileops_unary_fwd(0, None, None, -1, 0, 0.0, 0.0, 0, None) == -2  # size
    assert lib.tileops_unary_fwd(0, None, None, 16, 0, 0.0, 0.0, 0, None) == -3  # null
    assert lib.tileops_unary_fwd(0, None, None, 0, 0, 0.0, 0.0, 0, None) == 0    # empty
    assert lib.tileops_isfp_fwd(5, None, None, 16, 0, None) == -1
    assert lib.tileops_gated_gelu_fwd(3, None, None, 4, 4, 0, None) == -1
    assert lib.tileops_logsumexp_fwd(None, None, 4, 0, 0, None) == -2
    assert lib.tileops_argreduce_fwd(None, None, 0, 8, 0, 0, None) == 0
    assert lib.tileops_fused_add_layernorm_fwd(None, None, None, None, None, None, 4, 8, 1e-5,
                                               2, 1, None) == -1  # fp16 params for bf16 x
    # causal attention with more queries than keys (the right-aligned mask
    # would leave whole query blocks without a key) is rejected, as the Op does
    assert lib.tileops_mha_fwd(None, None, None, None, None, 1, 333, 200, 2, 2, 128, 1, 1.0,
                               0.0, 2, None) == -2
    assert lib.tileops_mha_fwd(None, None, None, None, None, 1, 333, 200, 2, 2, 128, 0, 1.0,
                               0.0, 2, None) == -3  # non-causal: fine until the null pointers
    assert lib.tileops_bitwise_not_fwd(None, None, -1, 0, None) == -2
    assert lib.tileops_bitwise_not_fwd(None, None, 0, 0, None) == 0
    assert lib.tileops_bitwise_not_fwd(None, None, 16, 1, None) == -3
    # GLA decode: positive sizes and scale, then the null pointers
    assert lib.tileops_gla_decode_fwd(None, None, None, None, None, None, None, 1, 2, 0, 64,
                                      0.1, 1, None) == -2
    assert lib.tileops_gla_decode_fwd(None, None, None, None, None, None, None, 1, 2, 64, 64,
                                      -1.0, 1, None) == -1
    assert lib.tileops_gla_decode_fwd(None, None, None, None, None, None, None, 1, 2, 64, 64,
                                      0.1, 1, None) == -3
    # GDN decode: DK / DV multiples of 32 (DK <= 256), a finite scale, then the
    # null pointers, then the 16-byte alignment of the states
    gdnd = lib.tileops_gdn_decode_fwd
    assert gdnd(None, None, None, None, None, None, None, None, 1, 2, 48, 64, 0.1, 2, None) == -2
    assert gdnd(None, None, None, None, None, None, None, None, 1, 2, 288, 64, 0.1, 2, None) == -2
    assert gdnd(None, None, None, None, None, None, None, None, 1, 2, 64, 80, 0.1, 2, None) == -2
    assert gdnd(None, None, None, None, None, None, None, None, 0, 2, 64, 64, 0.1, 2, None) == -2
    assert gdnd(None, None, None, None, None, None, None, None, 1 << 20, 1 << 20, 64, 64, 0.1, 2,
                None) == -2  # more workgroups than a grid holds
    assert gdnd(None, None, None, None, None, None, None, None, 1, 2, 64, 64,
                float("nan"), 2, None) == -1
    assert gdnd(None, None, None, None, None, None, None, None, 1, 2, 64, 64, 0.1, 2, None) == -3
    p = 4096  # non-null host values: the alignment test reads only the address
    assert gdnd(p, p, p, p, p, p + 4, p, p, 1, 2, 64, 64, 0.1, 2, None) == -1
    # softcap: 0 is off, positive caps; negative, NaN and infinite are rejected
    assert lib.tileops_mha_fwd(None, None, None, None, None, 1, 64, 64, 2, 2, 128, 0, 1.0,
                               30.0, 2, None) == -3
    for bad in (-1.0, float("nan"), float("inf")):
        assert lib.tileops_mha_fwd(None, None, None, None, None, 1, 64, 64, 2, 2, 128, 0, 1.0,
                                   bad, 2, None) == -1, bad
