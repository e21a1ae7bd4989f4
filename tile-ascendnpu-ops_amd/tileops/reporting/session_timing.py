"""Optional per-operator session timing attached to a run document.

Names and file contract of the reference's
examples/TileOPs/tileops/reporting/session_timing.py (imported by
tests/reporting/test_reporting.py:11; ``--with-session-timing`` on ``run``
and ``render``, cli.py:73-94).  A timing source is a Markdown file named
``SESSION_TIMING_ANALYSIS.md`` whose machine-readable part is one HTML
comment::

    <!-- TILEOPS_SESSION_TIMING_V1
    {"schema_version": 1, "operator": "...", "total_duration_s": 3661.25,
     "breakdown": [{"name": "...", "duration_s": 61.25, "ratio_percent": 1.67,
                    "detail": "..."}]}
    -->

Sources are found next to the package root through ``op_slug`` directories
named by ``.migration_meta.json`` files (``{"op_name", "op_slug"}``) under
``tileops/kernels``.  The section is rendered only when it was enabled;
with it off, a run document and its reports are unchanged.
"""

from __future__ import annotations

import json
import re
from pathlib import Path
from typing import Any, Iterable, Optional

__all__ = ["SOURCE_NAME", "attach_session_timing", "format_duration", "parse_session_timing"]

SOURCE_NAME = "SESSION_TIMING_ANALYSIS.md"
_BLOCK = re.compile(r"<!--\s*TILEOPS_SESSION_TIMING_V1\s*(\{.*?\})\s*-->", re.S)


def _record(status: str, operator: str, reason: Optional[str] = None,
            total: Optional[float] = None, breakdown: Optional[list] = None,
            source: Optional[Path] = None) -> dict[str, Any]:
    rec: dict[str, Any] = {"status": status, "operator": operator, "total_duration_s": total,
                           "breakdown": breakdown or []}
    if source is not None:
        rec["source"] = str(source)
    if reason:
        rec["reason"] = reason
    return rec


def _number(v: Any) -> Optional[float]:
    if isinstance(v, bool) or not isinstance(v, (int, float)):
        return None
    v = float(v)
    return v if v >= 0 and v == v and v != float("inf") else None


def parse_session_timing(path: str | Path, operator: str) -> dict[str, Any]:
    """The timing record of ``operator`` in the source file ``path``:
    ``status`` "available", "missing" (no file) or "invalid" (no block, bad
    JSON or schema, another operator, a negative or non-numeric duration),
    with ``reason`` for the last two."""
    path = Path(path)
    if not path.is_file():
        return _record("missing", operator, f"{SOURCE_NAME} not found")
    m = _BLOCK.search(path.read_text(encoding="utf-8"))
    if m is None:
        return _record("invalid", operator, "no TILEOPS_SESSION_TIMING_V1 block", source=path)
    try:
        doc = json.loads(m.group(1))
    except json.JSONDecodeError as exc:
        return _record("invalid", operator, f"malformed timing JSON: {exc.msg}", source=path)
    if doc.get("schema_version") != 1:
        return _record("invalid", operator,
                       f"unsupported schema_version {doc.get('schema_version')!r}", source=path)
    if doc.get("operator") != operator:
        return _record("invalid", operator,
                       f"operator mismatch: file names {doc.get('operator')!r}", source=path)
    total = _number(doc.get("total_duration_s"))
    if total is None:
        return _record("invalid", operator, "total_duration_s must be a non-negative number",
                       source=path)
    rows = []
    for item in doc.get("breakdown") or []:
        dur = _number(item.get("duration_s")) if isinstance(item, dict) else None
        if dur is None or not str(item.get("name", "")).strip():
            return _record("invalid", operator, "breakdown rows need a name and a duration_s",
                           source=path)
        ratio = _number(item.get("ratio_percent"))
        rows.append({"name": str(item["name"]), "duration_s": dur,
                     "ratio_percent": ratio if ratio is not None else
                     (100.0 * dur / total if total else None),
                     "detail": str(item.get("detail", ""))})
    return _record("available", operator, total=total, breakdown=rows, source=path)


def _slugs(root: Path) -> dict[str, str]:
    """op_name -> op_slug from every ``.migration_meta.json`` under tileops/kernels."""
    out: dict[str, str] = {}
    kernels = root / "tileops" / "kernels"
    if not kernels.is_dir():
        return out
    for meta in sorted(kernels.rglob(".migration_meta.json")):
        try:
            doc = json.loads(meta.read_text(encoding="utf-8"))
        except (OSError, json.JSONDecodeError):
            continue
        if isinstance(doc, dict) and doc.get("op_name") and doc.get("op_slug"):
            out.setdefault(str(doc["op_name"]), str(doc["op_slug"]))
    return out


def _candidates(root: Path, slug: Optional[str], kernel: Optional[str]) -> Iterable[Path]:
    if slug:
        yield root.parent / slug / SOURCE_NAME
        yield root / slug / SOURCE_NAME
    if kernel:
        yield (root / kernel).parent / SOURCE_NAME


def attach_session_timing(run: dict[str, Any], *, root: str | Path,
                          operator_catalog: Optional[list] = None,
                          enabled: bool = False) -> dict[str, Any]:
    """Add ``run["session_timing"] = {"enabled": True, "operators": {...}}``
    with one record per operator of the run; does nothing when disabled."""
    if not enabled:
        return run
    root = Path(root)
    slugs = _slugs(root)
    kernels = {c.get("name"): c.get("kernel") for c in operator_catalog or [] if c.get("name")}
    records: dict[str, Any] = {}
    for op in run.get("operators") or []:
        name = op.get("operator")
        if not name:
            continue
        found = next((p for p in _candidates(root, slugs.get(name), kernels.get(name))
                      if p.is_file()), None)
        records[name] = (parse_session_timing(found, name) if found is not None
                         else _record("missing", name, f"{SOURCE_NAME} not found"))
    run["session_timing"] = {"enabled": True, "operators": records}
    return run


def format_duration(seconds: Optional[float]) -> str:
    """``3661.25`` -> ``1h01m01s``; ``None`` -> ``N/A``."""
    if seconds is None:
        return "N/A"
    s = int(round(seconds))
    h, rem = divmod(s, 3600)
    m, sec = divmod(rem, 60)
    if h:
        return f"{h}h{m:02d}m{sec:02d}s"
    if m:
        return f"{m}m{sec:02d}s"
    return f"{sec}s"
