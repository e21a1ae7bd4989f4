"""Operator manifest: one YAML mapping per family, merged into one table.

Interface of the reference's loader (examples/TileOPs/tileops/manifest/__init__.py:18-89):
``manifest_files``, ``load_manifest`` (cached; a name defined in two files is
an error), ``load_workloads(op)`` (``KeyError`` for an unknown op),
``WORKLOAD_RESERVED_KEYS`` and ``single_input_workload_contract``.

Each entry carries ``signature``, ``workloads`` (the shapes every test and
benchmark runs), ``roofline`` (closed-form flop / byte expressions, evaluated
by :mod:`tileops.manifest.roofline`) and ``source`` (paths relative to the
project root: the kernel, op, test and benchmark files; ``test_keyword`` is
the ``pytest -k`` expression that selects the op's cases when one test file
covers several ops).
"""

from __future__ import annotations

import functools
from pathlib import Path
from typing import Any

import yaml

_DIR = Path(__file__).resolve().parent

WORKLOAD_RESERVED_KEYS: frozenset[str] = frozenset({"dtypes", "label"})


def manifest_files() -> list[Path]:
    """The family YAML files of the manifest, in name order."""
    return sorted(p for p in _DIR.iterdir() if p.is_file() and p.suffix == ".yaml")


@functools.lru_cache(maxsize=1)
def load_manifest() -> dict[str, Any]:
    """All entries of all family files, keyed by op name (cached)."""
    table: dict[str, Any] = {}
    where: dict[str, str] = {}
    for path in manifest_files():
        data = yaml.safe_load(path.read_text(encoding="utf-8")) or {}
        if not isinstance(data, dict):
            raise ValueError(
                f"manifest file {path.name} must contain a top-level mapping, "
                f"got {type(data).__name__}"
            )
        for name, entry in data.items():
            if name in table:
                raise ValueError(
                    f"duplicate op {name!r} in {path.name} (already defined in {where[name]})"
                )
            table[name] = entry
            where[name] = path.name
    return table


def load_workloads(op_name: str) -> list[dict[str, Any]]:
    """The ``workloads`` list of ``op_name``."""
    table = load_manifest()
    if op_name not in table:
        raise KeyError(f"op '{op_name}' not found in ops manifest")
    return table[op_name]["workloads"]


def single_input_workload_contract(
    signature: dict[str, Any],
) -> tuple[str, frozenset[str]] | None:
    """``(shape_key, allowed_keys)`` of a one-tensor-input op, else ``None``.

    The shape key is ``<input>_shape``; a workload may also name the op's
    params and the reserved keys."""
    if not isinstance(signature, dict):
        return None
    inputs = signature.get("inputs")
    if not isinstance(inputs, dict) or len(inputs) != 1:
        return None
    name = next(iter(inputs))
    if not isinstance(name, str):
        return None
    params = signature.get("params")
    names = frozenset(k for k in params if isinstance(k, str)) if isinstance(params, dict) else frozenset()
    shape_key = f"{name}_shape"
    return shape_key, names | WORKLOAD_RESERVED_KEYS | {shape_key}


__all__ = [
    "WORKLOAD_RESERVED_KEYS",
    "load_manifest",
    "load_workloads",
    "manifest_files",
    "single_input_workload_contract",
]
