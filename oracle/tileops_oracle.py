"""CPU oracle for the TileOPs forward-operator path -- TEST INFRASTRUCTURE ONLY.

This module restates, in numpy (float32 opmath, float64 only where stated),
the reference programs that define each operator's result in
Yihuace/tile-ascendnpu-ops; the HIP kernels' results are compared against
it.  Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg
may import it; the product path (tileops.*) never does.

Storage types are modelled explicitly: a tensor is a float32 numpy array
whose values are exactly representable in its storage dtype, and
``round_to(dtype, v)`` applies the round-to-nearest-even cast that torch's
``.to(dtype)`` performs.  bfloat16 rounding is done on the IEEE bit pattern.

Pins (tests/test_oracle_pins.py): every function is checked against torch's
CPU library routines on random and special-value inputs, against the
boundary cases the reference kernels' own harnesses hold, and against
closed forms; the GDN recurrence is additionally checked against an
independent chunked restatement and algebraic invariants.
"""

from __future__ import annotations

import math

import numpy as np

try:  # scipy provides a correctly rounded float erf; it is in the image
    from scipy.special import erf as _erf
except ImportError:  # pragma: no cover - scipy absent
    _erf = np.vectorize(math.erf, otypes=[np.float64])

F32, F16, BF16 = "float32", "float16", "bfloat16"


# ---------------------------------------------------------------------------
# storage-type rounding
# ---------------------------------------------------------------------------
def bf16_round(v: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 (nearest even), returned as float32."""
    v = np.ascontiguousarray(v, dtype=np.float32)
    u = v.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    out = r.view(np.float32).copy()
    nan = np.isnan(v)
    out[nan] = np.float32("nan")
    return out


def round_to(dtype: str, v) -> np.ndarray:
    v = np.asarray(v, dtype=np.float32)
    if dtype == F32:
        return v.copy()
    if dtype == F16:
        with np.errstate(over="ignore"):
            return v.astype(np.float16).astype(np.float32)
    if dtype == BF16:
        return bf16_round(v)
    raise ValueError(dtype)


# ---------------------------------------------------------------------------
# unary activations / clamp
# ---------------------------------------------------------------------------
def hardswish(x: np.ndarray, dtype: str) -> np.ndarray:
    """F.hardswish(x.float()).to(dtype) -- tests/ops/test_hardswish.py:38-39.
    x * min(max(x + 3, 0), 6) / 6 with NaN propagating through the clamp."""
    x = np.asarray(x, np.float32)
    t = x + np.float32(3)
    t = np.where(t < 0, np.float32(0), t)
    t = np.where(t > 6, np.float32(6), t)
    with np.errstate(invalid="ignore", over="ignore"):
        return round_to(dtype, x * t / np.float32(6))


def hardsigmoid(x: np.ndarray, dtype: str) -> np.ndarray:
    """F.hardsigmoid(x.float()).to(dtype) -- tests/ops/test_hardsigmoid.py:38-39."""
    x = np.asarray(x, np.float32)
    t = x + np.float32(3)
    t = np.where(t < 0, np.float32(0), t)
    t = np.where(t > 6, np.float32(6), t)
    return round_to(dtype, t / np.float32(6))


def add(a: np.ndarray, b: np.ndarray, alpha, dtype: str) -> np.ndarray:
    """torch.add(a, b, alpha=alpha) for half / fp32 storage: numpy broadcasting,
    fp32 opmath fma(alpha, b, a) -- torch's CPU kernel fuses the multiply-add --
    then rounded to the storage dtype (torch.sub is alpha -> -alpha).  The fma is
    the fp64 sum of the exact fp64 product (a 24x24-bit product fits in 53 bits)
    rounded to fp32."""
    a64 = np.asarray(a, np.float32).astype(np.float64)
    b64 = np.asarray(b, np.float32).astype(np.float64)
    y = a64 + np.float64(np.float32(alpha)) * b64
    return round_to(dtype, y.astype(np.float32))


def lerp(a: np.ndarray, b: np.ndarray, w, dtype: str) -> np.ndarray:
    """torch.lerp(a, b, w) for half / fp32 storage (tests/ops/test_lerp_scalar.py:58-60,
    test_lerp_tensor.py; the golden is torch.lerp itself): numpy broadcasting of
    a, b and a scalar or array weight, fp32 opmath d = b - a (rounded to fp32),
    then torch's two-sided form -- a + w d when |w| < 0.5, else b - (1 - w) d,
    each side one fused multiply-add (torch's vectorised CPU kernel, and its
    GPU kernel under contraction, fuse it) -- rounded to the storage dtype.
    The fma is emulated as the fp64 sum of the exact fp64 product, rounded to
    fp32 (it can differ from a true fma by one fp32 ulp in rare double-rounding
    cases)."""
    a32 = np.asarray(a, np.float32)
    b32 = np.asarray(b, np.float32)
    w32 = np.asarray(w, np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        d = (b32 - a32).astype(np.float32)
        small = np.abs(w32) < np.float32(0.5)
        coef = np.where(small, w32, (w32 - np.float32(1.0)).astype(np.float32))
        base = np.where(small, a32, b32)
        y = coef.astype(np.float64) * d.astype(np.float64) + base.astype(np.float64)
    return round_to(dtype, y.astype(np.float32))


def bitwise_not(x: np.ndarray) -> np.ndarray:
    """torch.bitwise_not(x) (tests/ops/test_bitwise_not.py of the reference):
    the complement of every integer, logical NOT of a bool."""
    x = np.asarray(x)
    return np.logical_not(x) if x.dtype == np.bool_ else np.invert(x)


def mish(x: np.ndarray, dtype: str) -> np.ndarray:
    """F.mish(x.float()).to(dtype) -- tests/ops/test_mish.py:38-39:
    x * tanh(log1p(exp(x))), fp64 arithmetic, rounded once."""
    xd = np.asarray(x, np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        y = xd * np.tanh(np.log1p(np.exp(xd)))
    return round_to(dtype, y.astype(np.float32))


def clamp_scalar(x: np.ndarray, dtype: str, lo=None, hi=None) -> np.ndarray:
    """torch.clamp(x.float(), min, max).to(dtype) -- tests/ops/test_clamp_scalar.py:56-57.
    NaN inputs propagate, a NaN bound gives NaN, min > max gives max."""
    if lo is None and hi is None:
        raise ValueError("present(min) or present(max)")
    y = np.asarray(x, np.float32).copy()
    nan_in = np.isnan(y)
    if lo is not None:
        lo32 = np.float32(lo)
        y = np.where(np.isnan(lo32) | (y < lo32), lo32, y)
    if hi is not None:
        hi32 = np.float32(hi)
        y = np.where(np.isnan(hi32) | (y > hi32), hi32, y)
    y = np.where(nan_in, np.float32("nan"), y)
    return round_to(dtype, y)


# ---------------------------------------------------------------------------
# float predicates (exact)
# ---------------------------------------------------------------------------
def isnan(x: np.ndarray) -> np.ndarray:
    """torch.isnan -- tests/ops/test_isnan.py:53-58."""
    return np.isnan(np.asarray(x, np.float32))


def isinf(x: np.ndarray) -> np.ndarray:
    """torch.isinf -- tests/ops/test_isinf.py:54-59."""
    return np.isinf(np.asarray(x, np.float32))


def isfinite(x: np.ndarray) -> np.ndarray:
    """torch.isfinite -- tests/ops/test_isfinite.py:55-60."""
    return np.isfinite(np.asarray(x, np.float32))


# ---------------------------------------------------------------------------
# gated GELU
# ---------------------------------------------------------------------------
def gelu_and_mul(x: np.ndarray, dtype: str) -> np.ndarray:
    """0.5 * g * (1 + erf(g * sqrt(0.5))) * v in fp32, cast once --
    tests/ops/test_gelu_and_mul.py:63-77 (gate = x[..., :N], value = x[..., N:])."""
    x = np.asarray(x, np.float32)
    half = x.shape[-1] // 2
    g, v = x[..., :half], x[..., half:]
    erf = _erf(g * np.float32(0.5**0.5)).astype(np.float32)
    gelu = np.float32(0.5) * g * (np.float32(1.0) + erf)
    return round_to(dtype, gelu * v)


def gelu_tanh_and_mul(x: np.ndarray, dtype: str) -> np.ndarray:
    """0.5 * g * (1 + tanh(sqrt(2/pi) * (g + 0.044715 g^3))) * v in fp32 --
    tests/ops/test_gelu_tanh_and_mul.py:64-81."""
    x = np.asarray(x, np.float32)
    half = x.shape[-1] // 2
    g, v = x[..., :half], x[..., half:]
    inner = np.float32(math.sqrt(2.0 / 3.141592653589793)) * (g + np.float32(0.044715) * g**3)
    gelu = np.float32(0.5) * g * (np.float32(1.0) + np.tanh(inner))
    return round_to(dtype, gelu * v)


# ---------------------------------------------------------------------------
# fused add + LayerNorm
# ---------------------------------------------------------------------------
def fused_add_layer_norm(x, residual, weight, bias, eps: float, dtype: str):
    """tests/ops/test_fused_add_layer_norm.py:55-72:
        added = (x.float() + residual.float()).to(dtype)
        y = F.layer_norm(added.float(), (n,), weight.float(), bias.float(), eps).to(dtype)
    Statistics: mean and biased variance of the rounded sum, accumulated in
    float64 here (torch accumulates fp32 in a different order; the final
    rounding to the storage type hides the difference)."""
    added = round_to(dtype, np.asarray(x, np.float32) + np.asarray(residual, np.float32))
    a64 = added.astype(np.float64)
    mean = a64.mean(axis=-1, keepdims=True)
    var = ((a64 - mean) ** 2).mean(axis=-1, keepdims=True)
    rstd = 1.0 / np.sqrt(var + eps)
    y = (a64 - mean) * rstd * np.asarray(weight, np.float64) + np.asarray(bias, np.float64)
    return round_to(dtype, y.astype(np.float32)), added


# ---------------------------------------------------------------------------
# reductions
# ---------------------------------------------------------------------------
def logsumexp(x: np.ndarray, dtype: str, axis: int = -1) -> np.ndarray:
    """torch.logsumexp(x.float(), dim).to(dtype) -- tests/ops/test_softmax.py:56-57.
    Shift by the row max unless it is infinite (then by 0): an all -inf row
    gives -inf, a row holding +inf gives +inf, NaN propagates.  float64 sum."""
    x = np.asarray(x, np.float32).astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        m = np.max(x, axis=axis, keepdims=True)
        m = np.where(np.isinf(m), 0.0, m)
        s = np.sum(np.exp(x - m), axis=axis, keepdims=True)
        y = np.log(s) + m
    return round_to(dtype, np.squeeze(y, axis=axis).astype(np.float32))


def argreduce(x: np.ndarray, axis: int = -1, is_min: bool = False) -> np.ndarray:
    """x.argmax(dim) / argmin -- tests/ops/test_argmax.py:163-165: the first index
    of the extreme value; any NaN is the extreme value (first NaN wins);
    -0.0 and +0.0 are equal."""
    x = np.moveaxis(np.asarray(x, np.float32), axis, -1)
    nan = np.isnan(x)
    any_nan = nan.any(axis=-1)
    first_nan = np.argmax(nan, axis=-1)
    clean = np.where(nan, np.float32(np.inf if is_min else -np.inf), x)
    ext = clean.min(axis=-1, keepdims=True) if is_min else clean.max(axis=-1, keepdims=True)
    first_ext = np.argmax(clean == ext, axis=-1)
    return np.where(any_nan, first_nan, first_ext).astype(np.int64)


# ---------------------------------------------------------------------------
# multi-head attention forward (BSHD)
# ---------------------------------------------------------------------------
def mha_fwd(q, k, v, is_causal: bool, dtype: str, scale: float | None = None,
            softcap: float = 0.0):
    """softmax(scale * q k^T [causal]) v per (b, h), plus the log2-domain LSE.
    With softcap > 0 the scaled scores are capped first, softcap *
    tanh(scores / softcap), then masked (golden_gqa_prefill_fwd,
    perf_opt/_gqa_prefill_fwd_kernel.py:180-186).

    Output: F.scaled_dot_product_attention on BHSD transposes
    (tests/ops/test_multi_head_attention.py:32-45); LSE: logsumexp(scores) / ln 2
    (tileops/kernels/attention/multi_head_attention/multi_head_attention_kernel/
    perf_opt/_gqa_prefill_fwd_kernel.py:151-194).  The causal mask is
    right-aligned: query i sees keys j <= i + (Skv - Sq).  fp64 math."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    B, Sq, H, D = q.shape
    Skv, Hkv = k.shape[1], k.shape[2]
    scale = D**-0.5 if scale is None else scale
    group = H // Hkv
    o = np.empty((B, Sq, H, D), np.float32)
    lse = np.empty((B, H, Sq), np.float32)
    if is_causal:
        qi = np.arange(Sq)[:, None] + (Skv - Sq)
        mask = np.arange(Skv)[None, :] > qi
    for b in range(B):
        for h in range(H):
            s = (q[b, :, h, :] @ k[b, :, h // group, :].T) * scale
            if softcap > 0.0:
                s = softcap * np.tanh(s / softcap)
            if is_causal:
                s = np.where(mask, -np.inf, s)
            m = s.max(axis=-1, keepdims=True)
            p = np.exp(s - m)
            den = p.sum(axis=-1, keepdims=True)
            o[b, :, h, :] = ((p / den) @ v[b, :, h // group, :]).astype(np.float32)
            lse[b, h] = ((np.log(den) + m)[:, 0] / math.log(2.0)).astype(np.float32)
    return round_to(dtype, o), lse


# ---------------------------------------------------------------------------
# gated linear attention (GLA) decode
# ---------------------------------------------------------------------------
def gla_decode(q, k, v, gk, state, scale: float, dtype: str):
    """One GLA decode step, restating golden_gla_decode
    (tileops/kernels/linear_attention/gla_decode/gla_decode_kernel/
    _gla_decode_kernel.py:211-218), layout BHD:

        new_state = exp(gk)[..., None] * state + k[..., None] * v[..., None, :]
        o         = scale * einsum("bhk,bhkv->bhv", q, new_state)

    fp64 arithmetic, the readout from the unrounded new state; both outputs
    rounded once to ``dtype``."""
    q, k, v, gk, s = (np.asarray(a, np.float64) for a in (q, k, v, gk, state))
    ns = np.exp(gk)[..., None] * s + k[..., :, None] * v[..., None, :]
    o = scale * np.einsum("bhk,bhkv->bhv", q, ns)
    return round_to(dtype, o.astype(np.float32)), round_to(dtype, ns.astype(np.float32))


# ---------------------------------------------------------------------------
# gated delta rule (GDN) prefill
# ---------------------------------------------------------------------------
def gdn_sequential(q, k, v, g, beta, h0, scale: float):
    """Token-by-token gated delta rule, restating golden_gdn_sequential
    (examples/gdn_prefill/probe/gdn_prefill_probe.py:60-77) for the BSHD layout:

        S <- S * exp(g_t)
        e  = beta_t * (v_t - k_t^T S)
        S <- S + k_t e^T
        o_t = scale * q_t^T S

    q, k: [B, T, H, K]; v: [B, T, H, V]; g, beta: [B, T, H]; h0: [B, H, K, V]
    or None.  float64 state.  Returns (o [B, T, H, V] float32, S [B, H, K, V] float32)."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    g = np.asarray(g, np.float64)
    beta = np.asarray(beta, np.float64)
    B, T, H, K = q.shape
    V = v.shape[-1]
    S = np.zeros((B, H, K, V)) if h0 is None else np.asarray(h0, np.float64).copy()
    o = np.empty((B, T, H, V))
    for t in range(T):
        S *= np.exp(g[:, t])[:, :, None, None]
        pred = np.einsum("bhk,bhkv->bhv", k[:, t], S)
        e = beta[:, t][:, :, None] * (v[:, t] - pred)
        S += k[:, t][:, :, :, None] * e[:, :, None, :]
        o[:, t] = scale * np.einsum("bhk,bhkv->bhv", q[:, t], S)
    return o.astype(np.float32), S.astype(np.float32)


def gdn_decode(q, k, v, g, beta, state, scale: float, dtype: str):
    """One decode step of the gated delta rule, layout BHD: the token step of
    golden_gdn_sequential (examples/gdn_prefill/probe/gdn_prefill_probe.py:60-77)
    on a single token,

        S  = exp(g) state
        e  = beta (v - k^T S)
        S' = S + k e^T
        o  = scale q^T S'

    q, k: [B, H, K]; v: [B, H, V]; g, beta: [B, H]; state: [B, H, K, V].
    float64 arithmetic; returns (o rounded once to ``dtype``, S' float32)."""
    q, k, v, g, beta = (np.asarray(a, np.float64) for a in (q, k, v, g, beta))
    S = np.exp(g)[:, :, None, None] * np.asarray(state, np.float64)
    e = beta[:, :, None] * (v - np.einsum("bhk,bhkv->bhv", k, S))
    S = S + k[:, :, :, None] * e[:, :, None, :]
    o = scale * np.einsum("bhk,bhkv->bhv", q, S)
    return round_to(dtype, o.astype(np.float32)), S.astype(np.float32)


def gdn_chunked(q, k, v, g, beta, h0, scale: float, chunk: int = 64):
    """The chunked form of the same recurrence (examples/gdn_prefill/DESIGN.md:6-17),
    used only to cross-check gdn_sequential.  Per chunk (local cumulative
    log-decay gc, decay matrix G[l,s] = exp(gc_l - gc_s) for l >= s):

        A   = strictly_lower(beta_l G[l,s] k_l.k_s)
        rhs = beta_l (v_l - exp(gc_l) k_l^T S)
        W   = (I + A)^-1 rhs                        (forward substitution)
        o_l = scale (exp(gc_l) q_l^T S + sum_{s<=l} G[l,s] (q_l.k_s) W_s)
        S  <- exp(gc_C) S + sum_l exp(gc_C - gc_l) k_l W_l^T
    float64 throughout."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    g = np.asarray(g, np.float64)
    beta = np.asarray(beta, np.float64)
    B, T, H, K = q.shape
    V = v.shape[-1]
    S = np.zeros((B, H, K, V)) if h0 is None else np.asarray(h0, np.float64).copy()
    o = np.empty((B, T, H, V))
    for b in range(B):
        for h in range(H):
            St = S[b, h]
            for c0 in range(0, T, chunk):
                sl = slice(c0, min(c0 + chunk, T))
                qc, kc, vc = q[b, sl, h], k[b, sl, h], v[b, sl, h]
                gc = np.cumsum(g[b, sl, h])
                bc = beta[b, sl, h]
                C = qc.shape[0]
                diff = gc[:, None] - gc[None, :]
                lower_incl = np.tril(np.ones((C, C), bool))
                G = np.where(lower_incl, np.exp(np.where(lower_incl, diff, 0.0)), 0.0)
                A = np.tril(bc[:, None] * G * (kc @ kc.T), -1)
                rhs = bc[:, None] * (vc - np.exp(gc)[:, None] * (kc @ St))
                W = np.empty_like(rhs)
                for i in range(C):
                    W[i] = rhs[i] - A[i, :i] @ W[:i]
                o[b, sl, h] = scale * (np.exp(gc)[:, None] * (qc @ St) + (G * (qc @ kc.T)) @ W)
                decay = np.exp(gc[-1] - gc)
                St = np.exp(gc[-1]) * St + (kc * decay[:, None]).T @ W
            S[b, h] = St
    return o.astype(np.float32), S.astype(np.float32)
