"""Evaluate a manifest entry's closed-form ``roofline`` block for one workload.

The block holds ``vars`` (evaluated in order), ``flops`` and ``bytes``:
Python expressions over the workload's keys, the op's param defaults from
``signature.params``, ``elem_bytes`` (the workload dtype's size),
``param_bytes`` (``param_dtype``'s size, default ``elem_bytes``) and the
helpers ``product`` and ``reduced_dims``.  The expressions come from this
package's own YAML files; they are evaluated with no builtins beyond the
few named here.
"""

from __future__ import annotations

import math
from typing import Any, Iterable

import torch

from tileops.manifest import WORKLOAD_RESERVED_KEYS, load_manifest

__all__ = ["manifest_roofline", "reduced_dims"]


def _broadcast(*shapes) -> tuple:
    """The broadcast shape of ``shapes`` (PyTorch / numpy rules)."""
    import numpy as np

    return tuple(np.broadcast_shapes(*(tuple(s) for s in shapes)))


def _product(values: Iterable[int]) -> int:
    return int(math.prod(int(v) for v in values))


def reduced_dims(shape, dim) -> list[int]:
    """Axes a reduction over ``dim`` covers: all of them for ``None``, else
    the (normalised, deduplicated) axes named."""
    nd = len(shape)
    if dim is None:
        return list(range(nd))
    if isinstance(dim, int):
        return [dim % nd]
    return sorted({d % nd for d in dim})


_SAFE = {
    "__builtins__": {},
    "product": _product,
    "broadcast": _broadcast,
    "reduced_dims": reduced_dims,
    "range": range,
    "len": len,
    "int": int,
    "min": min,
    "max": max,
    "isinstance": isinstance,
    "list": list,
    "tuple": tuple,
}


def _itemsize(dtype: Any) -> int:
    if isinstance(dtype, str):
        dtype = getattr(torch, dtype)
    return dtype.itemsize


def manifest_roofline(op_name: str, workload: dict[str, Any], dtype: Any) -> tuple[int, int]:
    """``(flops, bytes)`` of ``op_name``'s manifest formula at ``workload``
    (one row of its ``workloads``) computed in ``dtype``."""
    entry = load_manifest()[op_name]
    block = entry["roofline"]
    env: dict[str, Any] = {}
    params = (entry.get("signature") or {}).get("params") or {}
    for name, spec in params.items():
        if isinstance(spec, dict) and "default" in spec:
            env[name] = spec["default"]
    env.update({k: v for k, v in workload.items() if k not in WORKLOAD_RESERVED_KEYS})
    env["elem_bytes"] = _itemsize(dtype)
    env["param_bytes"] = _itemsize(workload.get("param_dtype", dtype))
    def _eval(expr: Any) -> Any:
        # names go into the globals so that comprehensions see them too
        return eval(str(expr), {**_SAFE, **env})  # noqa: S307 - package-owned formulas

    for name, expr in (block.get("vars") or {}).items():
        env[name] = _eval(expr)
    return int(_eval(block["flops"])), int(_eval(block["bytes"]))
