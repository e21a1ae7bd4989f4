"""Pin the CPU oracle before trusting it (runs without a GPU).

Each oracle function is checked against an independent source:
  * torch's CPU library routines (the reference programs call them),
  * exhaustive enumerations where the domain is small (every fp16 / bf16
    bit pattern for the predicates and the bf16 rounding),
  * the boundary cases of the reference kernels' own harnesses
    (hardswish_fwd_kernel.py:267-337, _logsumexp_kernel_single.py:215-224),
  * closed forms (uniform attention, delta-rule invariants),
chosen so that a dropped term, a wrong sign or a transposed operand fails.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import tileops_oracle as orc

DTYPES = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}


def _special_f32(n=4096, sigma=3.0, seed=0):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(n) * sigma).astype(np.float32)
    x[:24] = [0.0, -0.0, 3.0, -3.0, 6.0, -6.0, 2.999, -2.999, 1e-40, -1e-40, np.inf,
              -np.inf, np.nan, 65504.0, -65504.0, 3.4e38, -3.4e38, 1e-8, 0.5, -0.5,
              1.0, -1.0, 2.0, -2.0]
    return x


def _as_storage(x, dtype):
    return orc.round_to(dtype, x)


# -- storage rounding -------------------------------------------------------------
def test_bf16_round_matches_torch_on_all_upper_patterns():
    # every bf16 value plus values half-way between neighbours (ties to even)
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    vals = np.concatenate([hi, hi | 0x8000, hi | 0x7FFF, hi | 0x8001, hi | 0x1234])
    f = vals.view(np.float32)
    ref = torch.from_numpy(f.copy()).to(torch.bfloat16).float().numpy()
    got = orc.bf16_round(f)
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all()


def test_fp16_round_matches_torch():
    x = _special_f32(1 << 16)
    ref = torch.from_numpy(x).half().float().numpy()
    np.testing.assert_array_equal(orc.round_to("float16", x), ref)


# -- unary activations ---------------------------------------------------------------
@pytest.mark.parametrize("dtype", list(DTYPES))
@pytest.mark.parametrize("name", ["hardswish", "hardsigmoid"])
def test_activation_matches_torch_bitwise(name, dtype):
    x = _as_storage(_special_f32(), dtype)
    fn = F.hardswish if name == "hardswish" else F.hardsigmoid
    ref = fn(torch.from_numpy(x)).to(DTYPES[dtype]).float().numpy()
    got = getattr(orc, name)(x, dtype)
    np.testing.assert_array_equal(got, ref)  # NaN == NaN for assert_array_equal


def test_hardswish_boundary_cases():
    # reference harness: 0 -> 0, -3 -> -0.0, saturation, NaN / inf mapping
    x = np.array([0.0, -3.0, 3.0, 4.0, -4.0, 1.5, np.nan, np.inf, -np.inf], np.float32)
    y = orc.hardswish(x, "float32")
    assert y[0] == 0.0 and not np.signbit(y[0])
    assert y[1] == 0.0 and np.signbit(y[1])
    assert y[2] == 3.0 and y[3] == 4.0 and y[4] == 0.0
    assert y[5] == np.float32(1.5) * np.float32(4.5) / np.float32(6)
    assert np.isnan(y[6]) and y[7] == np.inf and np.isnan(y[8])
    s = orc.hardsigmoid(np.array([-3.0, 3.0, 0.0, np.nan, -np.inf, np.inf], np.float32), "float32")
    np.testing.assert_array_equal(s[:3], [0.0, 1.0, 0.5])
    assert np.isnan(s[3]) and s[4] == 0.0 and s[5] == 1.0


@pytest.mark.parametrize("dtype", list(DTYPES))
@pytest.mark.parametrize(
    "lo, hi", [(-0.5, 0.5), (None, 0.5), (-0.5, None), (-1.0, 1.0), (2.0, 1.0), (math.nan, 1.0),
               (0.0, math.nan)]
)
def test_clamp_matches_torch(dtype, lo, hi):
    x = _as_storage(_special_f32(), dtype)
    ref = torch.clamp(torch.from_numpy(x), lo, hi).to(DTYPES[dtype]).float().numpy()
    np.testing.assert_array_equal(orc.clamp_scalar(x, dtype, lo, hi), ref)


def test_clamp_requires_a_bound():
    with pytest.raises(ValueError, match="present"):
        orc.clamp_scalar(np.zeros(4, np.float32), "float32")


# -- predicates: every fp16 / bf16 encoding, fp32 special encodings ------------------
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_predicates_exhaustive_half(dtype):
    bits = torch.arange(1 << 16, dtype=torch.int32).to(torch.int16)
    x = bits.view(dtype)
    xf = x.float().numpy()
    for name in ("isnan", "isinf", "isfinite"):
        ref = getattr(torch, name)(x).numpy()
        np.testing.assert_array_equal(getattr(orc, name)(xf), ref)


def test_predicates_fp32_encodings():
    enc = np.array([0x7F800000, 0xFF800000, 0x7F800001, 0xFFC00000, 0x7FC00000, 0x7FFFFFFF,
                    0x00000001, 0x80000000, 0x7F7FFFFF, 0x3F800000], np.uint32)
    x = enc.view(np.float32)
    for name in ("isnan", "isinf", "isfinite"):
        ref = getattr(torch, name)(torch.from_numpy(x.copy())).numpy()
        np.testing.assert_array_equal(getattr(orc, name)(x), ref)


# -- gated GELU ------------------------------------------------------------------------
@pytest.mark.parametrize("approx", ["none", "tanh"])
def test_gated_gelu_matches_torch_gelu(approx):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((64, 2 * 96)) * 2).astype(np.float32)
    xt = torch.from_numpy(x)
    ref = (F.gelu(xt[:, :96], approximate=approx) * xt[:, 96:]).numpy()
    fn = orc.gelu_and_mul if approx == "none" else orc.gelu_tanh_and_mul
    np.testing.assert_allclose(fn(x, "float32"), ref, rtol=2e-6, atol=2e-6)


def test_gated_gelu_closed_forms():
    g = np.array([0.0, 8.0, -8.0, 1.0], np.float32)
    x = np.concatenate([g, np.full(4, 2.0, np.float32)])[None, :]
    y = orc.gelu_and_mul(x, "float32")[0]
    assert y[0] == 0.0 and y[1] == 16.0 and abs(y[2]) < 1e-12
    # gelu(1) = 0.5 (1 + erf(1/sqrt 2)) = Phi(1) = 0.8413447460685429
    assert abs(y[3] - 2 * 0.8413447460685429) < 1e-6
    yt = orc.gelu_tanh_and_mul(x, "float32")[0]
    assert yt[0] == 0.0 and yt[1] == 16.0 and abs(yt[2]) < 1e-10
    # 0.5 (1 + tanh(sqrt(2/pi) (1 + 0.044715)))
    assert abs(yt[3] - 2 * 0.8411919906082768) < 1e-6


# -- fused add + LayerNorm ------------------------------------------------------------
@pytest.mark.parametrize("dtype", list(DTYPES))
def test_layer_norm_matches_torch(dtype):
    rng = np.random.default_rng(2)
    m, n = 16, 1152
    x = _as_storage(rng.standard_normal((m, n)).astype(np.float32), dtype)
    r = _as_storage(rng.standard_normal((m, n)).astype(np.float32), dtype)
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    b = (0.1 * rng.standard_normal(n)).astype(np.float32)
    y, added = orc.fused_add_layer_norm(x, r, w, b, 1e-5, dtype)
    tdt = DTYPES[dtype]
    added_ref = (torch.from_numpy(x) + torch.from_numpy(r)).to(tdt)
    y_ref = F.layer_norm(added_ref.float(), (n,), torch.from_numpy(w), torch.from_numpy(b), 1e-5)
    np.testing.assert_array_equal(added, added_ref.float().numpy())
    tol = {"float32": 1e-5, "float16": 1e-3, "bfloat16": 1.6e-2}[dtype]
    np.testing.assert_allclose(y, y_ref.to(tdt).float().numpy(), rtol=tol, atol=tol)


def test_layer_norm_constant_row():
    # a constant row has zero variance: y = b exactly (rstd finite through eps)
    x = np.full((1, 64), 3.0, np.float32)
    y, added = orc.fused_add_layer_norm(x, np.zeros_like(x), np.full(64, 5.0, np.float32),
                                        np.arange(64, dtype=np.float32), 1e-5, "float32")
    np.testing.assert_array_equal(added, x)
    np.testing.assert_allclose(y[0], np.arange(64), atol=1e-6)


# -- reductions ------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", list(DTYPES))
def test_logsumexp_matches_torch(dtype):
    rng = np.random.default_rng(3)
    x = _as_storage((rng.standard_normal((33, 300)) * 2).astype(np.float32), dtype)
    x[0] = -np.inf
    x[1, 5] = np.inf
    x[2, 7] = np.nan
    x[3, :] = 88.0
    ref = torch.logsumexp(torch.from_numpy(x), dim=-1).to(DTYPES[dtype]).float().numpy()
    got = orc.logsumexp(x, dtype)
    assert got[0] == -np.inf and got[1] == np.inf and np.isnan(got[2])
    tol = {"float32": 1e-6, "float16": 1e-3, "bfloat16": 1.6e-2}[dtype]
    np.testing.assert_allclose(got, ref, rtol=tol, atol=tol)
    # closed form: a constant row c of length n -> c + ln n
    assert abs(orc.logsumexp(np.full((1, 300), 2.0, np.float32), "float32")[0]
               - (2.0 + math.log(300))) < 1e-6


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_logsumexp_huge_finite_rows(dtype):
    # finite maxima near the top of the range stay finite, as in torch
    big = float(torch.finfo(DTYPES[dtype]).max)
    rows = [[3e38, 0.0, 1.0], [-3e38, -3e38, -3e38], [big, big, 0.0], [-big, -big, -big],
            [3e38, -np.inf, np.inf], [-3e38, -np.inf, -np.inf], [3e38, np.nan, 1.0]]
    x = _as_storage(np.array(rows, np.float32), dtype)
    ref = torch.logsumexp(torch.from_numpy(x), dim=-1).to(DTYPES[dtype]).float().numpy()
    got = orc.logsumexp(x, dtype)
    assert np.isfinite(got[[0, 1, 2, 3, 5]]).all() and got[4] == np.inf and np.isnan(got[6])
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=0)


@pytest.mark.parametrize("is_min", [False, True])
def test_argreduce_matches_torch(is_min):
    rng = np.random.default_rng(4)
    x = rng.integers(-3, 4, size=(64, 97)).astype(np.float32)  # many ties
    x[0] = -np.inf
    x[1, [10, 40]] = np.nan
    x[2, :] = 0.0
    x[2, 5] = -0.0
    x[3, 50] = np.inf
    x[4, 60] = -np.inf
    t = torch.from_numpy(x)
    ref = (t.argmin(dim=-1) if is_min else t.argmax(dim=-1)).numpy()
    np.testing.assert_array_equal(orc.argreduce(x, -1, is_min), ref)
    assert orc.argreduce(x, -1, is_min)[1] == 10


def test_argmax_other_axis_and_flat():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4, 8, 16)).astype(np.float32)
    np.testing.assert_array_equal(orc.argreduce(x, 0), torch.from_numpy(x).argmax(0).numpy())
    assert orc.argreduce(x.reshape(1, -1), -1)[0] == torch.from_numpy(x).argmax().item()


def test_add_matches_torch():
    rng = np.random.default_rng(4)
    for sa, sb in (((6, 5), (6, 5)), ((4, 1, 3), (2, 1)), ((7,), ())):
        a = rng.standard_normal(sa).astype(np.float32)
        b = rng.standard_normal(sb).astype(np.float32)
        for dt, tdt in (("float32", torch.float32), ("float16", torch.float16),
                        ("bfloat16", torch.bfloat16)):
            ad, bd = orc.round_to(dt, a), orc.round_to(dt, b)
            ta, tb = torch.from_numpy(ad).to(tdt), torch.from_numpy(np.asarray(bd)).to(tdt)
            # the reference's golden: torch.add(a.float(), b.float(), alpha).to(dtype)
            # (tests/ops/test_add.py:68-69), torch.sub likewise
            for alpha in (1, 0.5, 3):
                want = torch.add(ta.float(), tb.float(), alpha=alpha).to(tdt).float().numpy()
                np.testing.assert_array_equal(orc.add(ad, bd, alpha, dt), want)
                want = torch.sub(ta.float(), tb.float(), alpha=alpha).to(tdt).float().numpy()
                np.testing.assert_array_equal(orc.add(ad, bd, -alpha, dt), want)


def _ulp_diff32(x, y):
    xi = np.asarray(x, np.float32).view(np.int32).astype(np.int64)
    yi = np.asarray(y, np.float32).view(np.int32).astype(np.int64)
    xi = np.where(xi < 0, -(xi & 0x7FFFFFFF), xi)
    yi = np.where(yi < 0, -(yi & 0x7FFFFFFF), yi)
    return np.abs(xi - yi)


def test_lerp_matches_torch():
    rng = np.random.default_rng(11)
    a = rng.standard_normal((64, 257)).astype(np.float32)
    b = (rng.standard_normal((64, 257)) * 3).astype(np.float32)
    wt = rng.uniform(-1.5, 2.5, (64, 257)).astype(np.float32)
    for dt, tdt in (("float32", torch.float32), ("float16", torch.float16),
                    ("bfloat16", torch.bfloat16)):
        ad, bd, wd = orc.round_to(dt, a), orc.round_to(dt, b), orc.round_to(dt, wt)
        ta, tb, tw = (torch.from_numpy(v).to(tdt) for v in (ad, bd, wd))
        # the reference's golden is torch.lerp on the storage dtype
        for w in (0.0, 0.3, 0.5, 0.7, 1.0, -1.5, 2.0):
            want = torch.lerp(ta, tb, w).float().numpy()
            got = orc.lerp(ad, bd, w, dt)
            if dt == "float32":
                assert _ulp_diff32(got, want).max() <= 1
            else:
                np.testing.assert_array_equal(got, want)
        want = torch.lerp(ta, tb, tw).float().numpy()
        got = orc.lerp(ad, bd, wd, dt)
        if dt == "float32":
            assert _ulp_diff32(got, want).max() <= 1
        else:
            np.testing.assert_array_equal(got, want)
    # broadcasting, as torch broadcasts
    a1 = rng.standard_normal((4, 1, 8)).astype(np.float32)
    b1 = rng.standard_normal((3, 1)).astype(np.float32)
    want = torch.lerp(torch.from_numpy(a1), torch.from_numpy(b1), 0.3).numpy()
    assert orc.lerp(a1, b1, 0.3, "float32").shape == want.shape == (4, 3, 8)
    assert _ulp_diff32(orc.lerp(a1, b1, 0.3, "float32"), want).max() <= 1


def test_lerp_closed_forms():
    rng = np.random.default_rng(12)
    a = rng.standard_normal(1000).astype(np.float32)
    b = rng.standard_normal(1000).astype(np.float32)
    # the endpoints are exact, whichever side of the formula computes them
    np.testing.assert_array_equal(orc.lerp(a, b, 0.0, "float32"), a)
    np.testing.assert_array_equal(orc.lerp(a, b, 1.0, "float32"), b)
    # the midpoint of two small integers is exact
    ia, ib = np.float32([1, -3, 8]), np.float32([4, 5, -2])
    np.testing.assert_array_equal(orc.lerp(ia, ib, 0.5, "float32"), (ia + ib) / 2)
    # a == b is a fixed point for every weight, and NaN propagates
    np.testing.assert_array_equal(orc.lerp(a, a, 0.37, "float32"), a)
    out = orc.lerp(np.float32([np.nan, 1.0]), np.float32([1.0, np.nan]), 0.25, "float32")
    assert np.isnan(out).all()


def test_mish_matches_torch():
    x = np.concatenate([np.linspace(-30, 30, 4001), [0.0, -0.0, 60.0, -60.0, 100.0, -100.0,
                                                      np.inf, -np.inf, np.nan]]).astype(np.float32)
    for dt, tdt in (("float32", torch.float32), ("float16", torch.float16),
                    ("bfloat16", torch.bfloat16)):
        xd = orc.round_to(dt, x)
        want = torch.nn.functional.mish(torch.from_numpy(xd)).to(tdt).float().numpy()
        got = orc.mish(xd, dt)
        assert np.array_equal(np.isnan(got), np.isnan(want)), dt
        ok = ~np.isnan(want)
        atol = {"float32": 1e-6, "float16": 1e-3, "bfloat16": 1e-2}[dt]
        np.testing.assert_allclose(got[ok], want[ok], rtol=atol, atol=atol, err_msg=dt)


# -- attention -----------------------------------------------------------------------
@pytest.mark.parametrize("causal", [False, True])
def test_mha_matches_sdpa(causal):
    rng = np.random.default_rng(6)
    B, S, H, D = 2, 40, 3, 16
    q, k, v = (rng.standard_normal((B, S, H, D)).astype(np.float32) for _ in range(3))
    o, lse = orc.mha_fwd(q, k, v, causal, "float32")
    tq, tk, tv = (torch.from_numpy(a).double().transpose(1, 2) for a in (q, k, v))
    ref = F.scaled_dot_product_attention(tq, tk, tv, is_causal=causal).transpose(1, 2)
    np.testing.assert_allclose(o, ref.float().numpy(), rtol=1e-5, atol=1e-6)
    s = (tq @ tk.transpose(-1, -2)) * D**-0.5
    if causal:
        s = s.masked_fill(torch.ones(S, S, dtype=torch.bool).triu(1), -math.inf)
    lse_ref = torch.logsumexp(s, -1) / math.log(2.0)
    np.testing.assert_allclose(lse, lse_ref.float().numpy(), rtol=1e-5, atol=1e-5)


def test_mha_uniform_attention_closed_form():
    # q = 0 -> every visible key has weight 1/n: o = running mean of v, lse = log2(n)
    B, S, H, D = 1, 9, 1, 4
    q = np.zeros((B, S, H, D), np.float32)
    k = np.ones((B, S, H, D), np.float32)
    v = np.arange(S * D, dtype=np.float32).reshape(B, S, H, D)
    o, lse = orc.mha_fwd(q, k, v, True, "float32")
    for i in range(S):
        np.testing.assert_allclose(o[0, i, 0], v[0, : i + 1, 0].mean(0), rtol=1e-6)
        assert abs(lse[0, 0, i] - math.log2(i + 1)) < 1e-6
    o, lse = orc.mha_fwd(q, k, v, False, "float32")
    np.testing.assert_allclose(o[0, :, 0], np.broadcast_to(v[0, :, 0].mean(0), (S, D)), rtol=1e-6)


def test_mha_softcap_limits_and_closed_forms():
    """Soft-capping (scores -> c tanh(scores / c), applied to the scaled scores
    before the mask, as golden_gqa_prefill_fwd does): a huge cap is the
    uncapped attention; one key gives lse = capped score / ln 2; two keys
    with scaled scores 2 and 0 under c = 1 weigh sigmoid(tanh 2) : 1 - that;
    a tiny cap flattens every row to uniform attention."""
    rng = np.random.default_rng(9)
    B, S, H, D = 1, 24, 2, 8
    q, k, v = (rng.standard_normal((B, S, H, D)).astype(np.float32) for _ in range(3))
    for causal in (False, True):
        o0, l0 = orc.mha_fwd(q, k, v, causal, "float32")
        o1, l1 = orc.mha_fwd(q, k, v, causal, "float32", softcap=1e6)
        np.testing.assert_allclose(o1, o0, rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(l1, l0, rtol=1e-5, atol=1e-6)
    # scale * q.k = 0.5 * 4 = 2 for the first key, 0 for the second
    q1 = np.ones((1, 1, 1, 4), np.float32)
    k2 = np.stack([np.ones(4), np.zeros(4)]).astype(np.float32).reshape(1, 2, 1, 4)
    v2 = np.array([[1.0, 0, 0, 0], [0, 1.0, 0, 0]], np.float32).reshape(1, 2, 1, 4)
    o, lse = orc.mha_fwd(q1, k2[:, :1], v2[:, :1], False, "float32", scale=0.5, softcap=1.0)
    assert abs(lse[0, 0, 0] - 0.9640275800758169 / math.log(2.0)) < 1e-6  # tanh(2)
    np.testing.assert_allclose(o[0, 0, 0], v2[0, 0, 0], rtol=1e-6)
    o, lse = orc.mha_fwd(q1, k2, v2, False, "float32", scale=0.5, softcap=1.0)
    w1 = 1.0 / (1.0 + math.exp(-0.9640275800758169))
    np.testing.assert_allclose(o[0, 0, 0], [w1, 1.0 - w1, 0.0, 0.0], rtol=1e-6, atol=1e-7)
    # tiny cap: every capped score within 1e-3 of 0 -> near-uniform rows
    o, lse = orc.mha_fwd(q, k, v, False, "float32", softcap=1e-3)
    np.testing.assert_allclose(o[0, :, 0], np.broadcast_to(v[0, :, 0].mean(0), (S, D)), atol=1e-3)
    np.testing.assert_allclose(lse, math.log2(S), atol=1e-2)


# -- GLA decode -------------------------------------------------------------------------
def test_gla_decode_closed_forms():
    """gk = 0 and a zero state leave new_state = k v^T and o = scale (q.k) v;
    k = 0 leaves a pure decay, new_state = e^gk state, read out as
    scale q^T (e^gk state); the two add up (the update is linear in the state
    and in k v^T)."""
    rng = np.random.default_rng(12)
    B, H, DK, DV, scale = 2, 3, 8, 5, 0.3
    q, k, gk = (rng.standard_normal((B, H, DK)) for _ in range(3))
    v = rng.standard_normal((B, H, DV))
    s0 = rng.standard_normal((B, H, DK, DV))
    o, ns = orc.gla_decode(q, k, v, np.zeros_like(gk), np.zeros_like(s0), scale, "float32")
    np.testing.assert_allclose(ns, np.einsum("bhk,bhv->bhkv", k, v), rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(o, scale * (q * k).sum(-1)[..., None] * v, rtol=1e-5, atol=1e-6)
    o2, ns2 = orc.gla_decode(q, np.zeros_like(k), v, gk, s0, scale, "float32")
    decayed = np.exp(gk)[..., None] * s0
    np.testing.assert_allclose(ns2, decayed, rtol=1e-6, atol=1e-6)
    want = scale * np.stack([[q[b, h] @ decayed[b, h] for h in range(H)] for b in range(B)])
    np.testing.assert_allclose(o2, want, rtol=1e-5, atol=1e-6)
    o3, ns3 = orc.gla_decode(q, k, v, gk, s0, scale, "float32")
    np.testing.assert_allclose(ns3, ns2 + np.einsum("bhk,bhv->bhkv", k, v), rtol=1e-5, atol=1e-6)


# -- gated delta rule -----------------------------------------------------------------
def _gdn_inputs(B=2, T=37, H=2, K=8, V=6, seed=7, h0=True):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, T, H, K))
    k = rng.standard_normal((B, T, H, K))
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    v = rng.standard_normal((B, T, H, V))
    g = np.log(1 / (1 + np.exp(-rng.standard_normal((B, T, H)))))  # logsigmoid
    beta = 1 / (1 + np.exp(-rng.standard_normal((B, T, H))))
    s0 = rng.standard_normal((B, H, K, V)) if h0 else None
    return q, k, v, g, beta, s0


@pytest.mark.parametrize("chunk", [4, 16, 64])
def test_gdn_sequential_equals_chunked(chunk):
    q, k, v, g, beta, s0 = _gdn_inputs()
    o1, s1 = orc.gdn_sequential(q, k, v, g, beta, s0, 0.3)
    o2, s2 = orc.gdn_chunked(q, k, v, g, beta, s0, 0.3, chunk=chunk)
    np.testing.assert_allclose(o1, o2, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(s1, s2, rtol=1e-5, atol=1e-5)


def test_gdn_beta_zero_only_decays():
    q, k, v, g, beta, s0 = _gdn_inputs()
    beta[:] = 0.0
    o, s = orc.gdn_sequential(q, k, v, g, beta, s0, 0.5)
    cum = np.cumsum(g, axis=1)  # [B, T, H]
    np.testing.assert_allclose(s, np.exp(cum[:, -1])[:, :, None, None] * s0, rtol=1e-5)
    expect = 0.5 * np.einsum("bthk,bhkv->bthv", q, s0) * np.exp(cum)[..., None]
    np.testing.assert_allclose(o, expect, rtol=1e-4, atol=1e-5)


def test_gdn_delta_rule_writes_values():
    # g = 0, beta = 1, orthonormal keys: the state maps each key to its value
    K = V = 8
    T = 6
    keys = np.linalg.qr(np.random.default_rng(8).standard_normal((K, K)))[0][:T]
    k = keys[None, :, None, :]
    v = np.random.default_rng(9).standard_normal((1, T, 1, V))
    z = np.zeros((1, T, 1))
    o, s = orc.gdn_sequential(k, k, v, z, np.ones((1, T, 1)), None, 1.0)
    np.testing.assert_allclose(keys @ s[0, 0], v[0, :, 0], atol=1e-6)
    np.testing.assert_allclose(o[0, :, 0], v[0, :, 0], atol=1e-6)  # q_t = k_t reads v_t


def test_gdn_empty_sequence_passes_state_through():
    q, k, v, g, beta, s0 = _gdn_inputs(T=0)
    o, s = orc.gdn_sequential(q, k, v, g, beta, s0, 1.0)
    assert o.shape == (2, 0, 2, 6)
    np.testing.assert_allclose(s, s0, rtol=1e-6)


def test_gdn_decode_steps_equal_the_sequential_recurrence():
    # T decode steps from h0 reproduce the token loop over the whole sequence
    q, k, v, g, beta, s0 = _gdn_inputs(T=5)
    o_seq, s_seq = orc.gdn_sequential(q, k, v, g, beta, s0, 0.3)
    s = s0.astype(np.float32)
    for t in range(q.shape[1]):
        o, s = orc.gdn_decode(q[:, t], k[:, t], v[:, t], g[:, t], beta[:, t], s, 0.3, "float32")
        np.testing.assert_allclose(o, o_seq[:, t], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(s, s_seq, rtol=1e-5, atol=1e-6)


def test_gdn_decode_closed_forms():
    *seq, s0 = _gdn_inputs(T=1)
    q, k, v, g, beta = (a[:, 0] for a in seq)
    # beta = 0: decay only, and the readout is exp(g) q^T state
    o, s = orc.gdn_decode(q, k, v, g, np.zeros_like(beta), s0, 0.5, "float32")
    np.testing.assert_allclose(s, np.exp(g)[:, :, None, None] * s0, rtol=1e-6)
    np.testing.assert_allclose(o, 0.5 * np.exp(g)[..., None] * np.einsum("bhk,bhkv->bhv", q, s0),
                               rtol=1e-5, atol=1e-6)
    # beta = 1 with a unit key: the new state reads v back at k
    o, s = orc.gdn_decode(k, k, v, g, np.ones_like(beta), s0, 1.0, "float32")
    np.testing.assert_allclose(np.einsum("bhk,bhkv->bhv", k, s), v, atol=1e-6)
    np.testing.assert_allclose(o, v, atol=1e-6)
    # directions orthogonal to k keep the decayed state
    u = np.random.default_rng(3).standard_normal(k.shape)
    u -= np.sum(u * k, -1, keepdims=True) * k
    np.testing.assert_allclose(np.einsum("bhk,bhkv->bhv", u, s),
                               np.exp(g)[..., None] * np.einsum("bhk,bhkv->bhv", u, s0),
                               rtol=1e-5, atol=1e-6)


# -- the torch reference programs bench.py times as the CPU baseline ---------------------
def test_torch_reference_programs_match_the_oracle():
    from oracle import torch_ref as tr

    rng = np.random.default_rng(21)
    x16 = torch.from_numpy((rng.standard_normal((64, 96)) * 3).astype(np.float32)).half()
    xn = x16.float().numpy()
    assert np.array_equal(tr.hardswish(x16).float().numpy(), orc.hardswish(xn, "float16"))
    assert np.array_equal(tr.hardsigmoid(x16).float().numpy(), orc.hardsigmoid(xn, "float16"))
    assert np.array_equal(tr.clamp_scalar(x16, -1.0, 1.0).float().numpy(),
                          orc.clamp_scalar(xn, "float16", -1.0, 1.0))
    xs = rng.standard_normal((32, 64)).astype(np.float32)
    xs[0, :3] = [np.nan, np.inf, -np.inf]
    for fn in ("isnan", "isinf", "isfinite"):
        assert np.array_equal(getattr(tr, fn)(torch.from_numpy(xs)).numpy(), getattr(orc, fn)(xs))
    xg = torch.from_numpy(rng.standard_normal((16, 256)).astype(np.float32)).bfloat16()
    for fn in ("gelu_and_mul", "gelu_tanh_and_mul"):
        np.testing.assert_allclose(getattr(tr, fn)(xg).float().numpy(),
                                   getattr(orc, fn)(xg.float().numpy(), "bfloat16"),
                                   rtol=1.6e-2, atol=1.6e-2)
    xl = torch.from_numpy(rng.standard_normal((8, 128)).astype(np.float32)).bfloat16()
    rl = torch.from_numpy(rng.standard_normal((8, 128)).astype(np.float32)).bfloat16()
    w = torch.from_numpy((1 + 0.1 * rng.standard_normal(128)).astype(np.float32))
    b = torch.from_numpy((0.1 * rng.standard_normal(128)).astype(np.float32))
    y, added = tr.fused_add_layer_norm(xl, rl, w, b, 1e-5)
    y_ref, added_ref = orc.fused_add_layer_norm(xl.float().numpy(), rl.float().numpy(),
                                                w.numpy(), b.numpy(), 1e-5, "bfloat16")
    assert np.array_equal(added.float().numpy(), added_ref)
    np.testing.assert_allclose(y.float().numpy(), y_ref, rtol=1.6e-2, atol=1.6e-2)
    xr = torch.from_numpy((rng.standard_normal((40, 300)) * 2).astype(np.float32))
    np.testing.assert_allclose(tr.logsumexp(xr).numpy(), orc.logsumexp(xr.numpy(), "float32"),
                               rtol=1e-5, atol=1e-5)
    assert np.array_equal(tr.argmax(xr).numpy(), orc.argreduce(xr.numpy(), -1))
    q, k, v = (torch.from_numpy(rng.standard_normal((1, 48, 2, 64)).astype(np.float32)).bfloat16()
               for _ in range(3))
    for causal in (False, True):
        o_ref, _ = orc.mha_fwd(q.float().numpy(), k.float().numpy(), v.float().numpy(), causal,
                               "bfloat16")
        np.testing.assert_allclose(tr.mha_fwd(q, k, v, causal).float().numpy(), o_ref,
                                   rtol=1e-2, atol=1e-2)


def test_torch_gdn_sequential_matches_the_oracle():
    from oracle import torch_ref as tr

    rng = np.random.default_rng(22)
    B, T, H, K, V = 1, 40, 2, 16, 8
    q = rng.standard_normal((B, T, H, K)).astype(np.float32)
    k = rng.standard_normal((B, T, H, K)).astype(np.float32)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((B, T, H, V)).astype(np.float32)
    g = -np.abs(rng.standard_normal((B, T, H))).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal((B, T, H))))).astype(np.float32)
    o, S = tr.gdn_sequential(*(torch.from_numpy(a) for a in (q, k, v, g, beta)), 0.25)
    o_ref, S_ref = orc.gdn_sequential(q, k, v, g, beta, None, 0.25)
    np.testing.assert_allclose(o.numpy(), o_ref, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(S.numpy(), S_ref, rtol=1e-4, atol=1e-5)
