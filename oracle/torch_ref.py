"""The reference's own reference programs, in torch on the CPU -- TEST
INFRASTRUCTURE ONLY.

Each function restates the ``ref_program`` (or golden) that a reference test
compares its operator against, as torch CPU code: what the reference suite
runs as ground truth, multi-threaded by torch's intra-op pool.  bench.py's
CPU-baseline leg times them beside the GPU kernels; tests/test_oracle_pins.py
checks each against the numpy oracle (oracle/tileops_oracle.py).  Nothing in
the product path imports this module.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def hardswish(x: torch.Tensor) -> torch.Tensor:
    """F.hardswish(x.float()).to(dtype) -- tests/ops/test_hardswish.py:38-39."""
    return F.hardswish(x.float()).to(x.dtype)


def hardsigmoid(x: torch.Tensor) -> torch.Tensor:
    """F.hardsigmoid(x.float()).to(dtype) -- tests/ops/test_hardsigmoid.py:38-39."""
    return F.hardsigmoid(x.float()).to(x.dtype)


def clamp_scalar(x: torch.Tensor, lo, hi) -> torch.Tensor:
    """torch.clamp(x.float(), min, max).to(dtype) -- tests/ops/test_clamp_scalar.py:56-57."""
    return torch.clamp(x.float(), lo, hi).to(x.dtype)


def isnan(x: torch.Tensor) -> torch.Tensor:
    """torch.isnan(x.float()) -- tests/ops/test_isnan.py:53-58."""
    return torch.isnan(x.float())


def isinf(x: torch.Tensor) -> torch.Tensor:
    """torch.isinf(x.float()) -- tests/ops/test_isinf.py:54-59."""
    return torch.isinf(x.float())


def isfinite(x: torch.Tensor) -> torch.Tensor:
    """torch.isfinite(x.float()) -- tests/ops/test_isfinite.py:55-60."""
    return torch.isfinite(x.float())


def gelu_and_mul(x: torch.Tensor) -> torch.Tensor:
    """0.5 g (1 + erf(g / sqrt 2)) v in fp32, cast once -- tests/ops/test_gelu_and_mul.py:63-77."""
    n = x.shape[-1] // 2
    g, v = x[..., :n].float(), x[..., n:].float()
    return (0.5 * g * (1.0 + torch.erf(g / math.sqrt(2.0))) * v).to(x.dtype)


def gelu_tanh_and_mul(x: torch.Tensor) -> torch.Tensor:
    """0.5 g (1 + tanh(sqrt(2/pi) (g + 0.044715 g^3))) v in fp32 --
    tests/ops/test_gelu_tanh_and_mul.py:64-81."""
    n = x.shape[-1] // 2
    g, v = x[..., :n].float(), x[..., n:].float()
    u = math.sqrt(2.0 / math.pi) * (g + 0.044715 * g * g * g)
    return (0.5 * g * (1.0 + torch.tanh(u)) * v).to(x.dtype)


def fused_add_layer_norm(x, residual, weight, bias, eps: float):
    """residual_out = (x + residual) rounded to the dtype, y = layer_norm of it in
    fp32 -- tests/ops/test_fused_add_layer_norm.py:55-72."""
    added = (x.float() + residual.float()).to(x.dtype)
    y = F.layer_norm(added.float(), (x.shape[-1],), weight.float(), bias.float(), eps)
    return y.to(x.dtype), added


def logsumexp(x: torch.Tensor, dim: int = -1) -> torch.Tensor:
    """torch.logsumexp(x.float(), dim).to(dtype) -- tests/ops/test_softmax.py:56-57."""
    return torch.logsumexp(x.float(), dim).to(x.dtype)


def argmax(x: torch.Tensor, dim: int = -1) -> torch.Tensor:
    """x.argmax(dim) -- tests/ops/test_argmax.py:163-165."""
    return x.argmax(dim=dim)


def mha_fwd(q, k, v, is_causal: bool):
    """F.scaled_dot_product_attention on BHSD transposes of BSHD inputs, in
    fp32 -- tests/ops/test_multi_head_attention.py:32-45."""
    qb, kb, vb = (t.float().transpose(1, 2) for t in (q, k, v))
    o = F.scaled_dot_product_attention(qb, kb, vb, is_causal=is_causal)
    return o.transpose(1, 2).to(q.dtype)


def gdn_sequential(q, k, v, g, beta, scale: float, h0=None):
    """Token-by-token gated delta rule, golden_gdn_sequential
    (examples/gdn_prefill/probe/gdn_prefill_probe.py:60-77), BSHD layout,
    every (batch, head) in one batched step per token, fp32 state."""
    q, k, v = q.float(), k.float(), v.float()
    B, T, H, K = q.shape
    V = v.shape[-1]
    S = torch.zeros(B, H, K, V) if h0 is None else h0.float().clone()
    o = torch.empty(B, T, H, V)
    for t in range(T):
        S.mul_(torch.exp(g[:, t].float())[:, :, None, None])
        pred = torch.einsum("bhk,bhkv->bhv", k[:, t], S)
        e = beta[:, t].float()[:, :, None] * (v[:, t] - pred)
        S.add_(k[:, t][:, :, :, None] * e[:, :, None, :])
        o[:, t] = scale * torch.einsum("bhk,bhkv->bhv", q[:, t], S)
    return o, S
