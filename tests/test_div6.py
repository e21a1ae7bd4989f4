"""The kernels' division by 6 (hardswish, hardsigmoid) is correctly rounded.

The device computes n / 6 as q0 = RN(n RN(1/6)), e = RN(n - 6 q0) (exact),
q = RN(q0 + e RN(1/6)), keeping q0 when e == 0 or q0 is not finite.  This
restates that sequence with exact rational arithmetic and compares it with
the correctly rounded float32 quotient (numpy division) for every numerator
the two ops produce from all fp16 and bf16 encodings, plus fp32 stress values.
"""

from fractions import Fraction

import numpy as np
import pytest

R6 = np.float32(1.0) / np.float32(6.0)  # RN(1/6) = 0x3E2AAAAB


def _rn32(x: Fraction) -> np.float32:
    """Round an exact rational to the nearest float32 (ties to even)."""
    if x == 0:
        return np.float32(0.0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, -126)  # subnormal range shares the minimum exponent
    scale = Fraction(2) ** (23 - e)
    m = a * scale
    fl = m.numerator // m.denominator
    rem = m - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    val = Fraction(fl) / scale
    if val >= Fraction(2) ** 128:
        return np.float32(sign * np.inf)
    return np.float32(sign * float(val))


def _div6_device(n: np.float32) -> np.float32:
    q0 = np.float32(n * R6)
    if not np.isfinite(q0):
        return q0
    e = _rn32(Fraction(float(n)) - 6 * Fraction(float(q0)))
    if e == 0:
        return q0
    return _rn32(Fraction(float(q0)) + Fraction(float(e)) * Fraction(float(R6)))


def _numerators(dtype) -> np.ndarray:
    bits = np.arange(65536, dtype=np.uint32)
    if dtype == "float16":
        x = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    else:
        x = (bits << 16).view(np.float32)
    x = x[np.isfinite(x)]
    t = np.clip(x + np.float32(3.0), np.float32(0.0), np.float32(6.0)).astype(np.float32)
    return np.unique(np.concatenate([x * t, t]).astype(np.float32))


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_div6_matches_division_on_all_half_numerators(dtype):
    ns = _numerators(dtype)
    want = ns / np.float32(6.0)
    for n, w in zip(ns, want):
        got = _div6_device(n)
        assert got == w and np.signbit(got) == np.signbit(w), (n, got, w)


def test_div6_fp32_stress_values():
    rng = np.random.default_rng(1235)
    vals = [0.0, -0.0, 6.0, -6.0, 1e-45, -1e-45, 1.1754944e-38, 3.4028235e38, -3.4028235e38,
            np.float32(1.0) / np.float32(3.0), 7.0, 1e-40]
    vals += list(rng.standard_normal(4000).astype(np.float32) * np.float32(8.0))
    vals += list((rng.integers(1, 2**31, 2000, dtype=np.int64).astype(np.uint32)).view(np.float32))
    for v in np.array(vals, dtype=np.float32):
        if not np.isfinite(v):
            continue
        want = np.float32(v / np.float32(6.0))
        got = _div6_device(v)
        assert got == want and np.signbit(got) == np.signbit(want), (v, got, want)
