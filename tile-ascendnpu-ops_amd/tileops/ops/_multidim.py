"""Multi-dim reduction shape helpers (device independent).

Same contract as the reference's examples/TileOPs/tileops/ops/_multidim.py:22-94:
``normalize_dim`` canonicalises and validates dims, ``flatten_for_multidim``
moves the reduced dims last and flattens to ``[*kept, reduced]``, and
``restore_multidim_shape`` maps the ``(M,)`` result back.
"""

from __future__ import annotations

from typing import Literal, Union

import torch

__all__ = ["EmptyDimPolicy", "flatten_for_multidim", "normalize_dim", "restore_multidim_shape"]

EmptyDimPolicy = Literal["reject", "full", "noop"]


def normalize_dim(
    dim: Union[int, list[int], None],
    ndim: int,
    *,
    empty_dim_policy: EmptyDimPolicy = "reject",
) -> list[int]:
    if dim is None:
        return list(range(ndim))
    dims = [dim] if isinstance(dim, int) else list(dim)
    if not dims:
        if empty_dim_policy == "full":
            return list(range(ndim))
        if empty_dim_policy == "noop":
            return []
        raise ValueError(
            "dim=[] is not supported by this op; pass "
            'empty_dim_policy="full" to opt in to full-reduction '
            'or empty_dim_policy="noop" to opt in to the identity contract.'
        )
    out = []
    for d in dims:
        if d < -ndim or d >= ndim:
            raise IndexError(
                f"Dimension out of range (expected to be in range of "
                f"[{-ndim}, {ndim - 1}], but got {d})"
            )
        out.append(d % ndim)
    if len(set(out)) != len(out):
        raise ValueError(f"Duplicate dims in reduction: {dims}")
    return sorted(out)


def flatten_for_multidim(
    x: torch.Tensor, dims: list[int]
) -> tuple[torch.Tensor, torch.Size, list[int]]:
    orig_shape = x.shape
    kept = [i for i in range(x.ndim) if i not in dims]
    x = x.permute(kept + list(dims)).contiguous()
    kept_shape = [orig_shape[i] for i in kept]
    reduced = 1
    for d in dims:
        reduced *= orig_shape[d]
    return x.reshape(kept_shape + [reduced] if kept_shape else [1, reduced]), orig_shape, kept


def restore_multidim_shape(
    y: torch.Tensor, orig_shape: torch.Size, dims: list[int], keepdim: bool
) -> torch.Tensor:
    if keepdim:
        shape = list(orig_shape)
        for d in dims:
            shape[d] = 1
        return y.reshape(shape)
    shape = [orig_shape[i] for i in range(len(orig_shape)) if i not in dims]
    return y.squeeze() if not shape else y.reshape(shape)
