"""rocprofv3 kernel-time measurement of an Op rebuilt in a subprocess.

The subprocess reconstructs the Op from its constructor-named attributes
(the contract of the reference's examples/TileOPs/tileops/benchmark/msprof.py:108-139),
so Ops keep every ``__init__`` argument as an attribute of the same name.
"""

from __future__ import annotations

import inspect
from typing import Any

import torch

__all__ = ["_extract_op_init_args"]


def _is_serializable(val: Any) -> bool:
    if val is None or isinstance(val, (bool, int, float, str, torch.dtype)):
        return True
    if isinstance(val, (list, tuple)):
        return all(_is_serializable(v) for v in val)
    return False


def _extract_op_init_args(op: Any) -> dict:
    """Constructor arguments of ``op`` read back from its attributes.

    Walks ``type(op).__init__``'s named parameters and keeps those the
    instance holds under the same name with a plain serializable value
    (kernels, kernel maps and caches are skipped)."""
    try:
        sig = inspect.signature(type(op).__init__)
    except (TypeError, ValueError):
        return {}
    out: dict = {}
    for name, param in sig.parameters.items():
        if name == "self" or param.kind in (param.VAR_POSITIONAL, param.VAR_KEYWORD):
            continue
        if hasattr(op, name):
            val = getattr(op, name)
            if _is_serializable(val):
                out[name] = val
    return out
