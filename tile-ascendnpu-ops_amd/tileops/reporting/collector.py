"""Readers for pytest JUnit XML and the benchmark JSON.

Schemas of the reference's collector (examples/TileOPs/tileops/reporting/collector.py:18-100).
"""

from __future__ import annotations

import json
import xml.etree.ElementTree as ET
from pathlib import Path
from typing import Any

_EMPTY_COUNTS = {"tests": 0, "passed": 0, "failed": 0, "errors": 0, "skipped": 0}


def _int(value: str | None) -> int:
    try:
        return int(value or 0)
    except ValueError:
        return 0


def _case(node: ET.Element) -> dict[str, Any]:
    outcome, message = "passed", None
    for tag in ("failure", "error", "skipped"):
        child = node.find(tag)
        if child is not None:
            outcome = "failed" if tag == "failure" else tag
            message = child.get("message") or (child.text or "").strip() or None
            break
    props = {p.get("name", ""): p.get("value", "")
             for p in node.findall("./properties/property") if p.get("name")}
    classname, name = node.get("classname", ""), node.get("name", "")
    return {
        "nodeid": "::".join(x for x in (classname, name) if x),
        "name": name,
        "classname": classname,
        "time_s": float(node.get("time", "0") or 0),
        "outcome": outcome,
        "message": message,
        "properties": props,
    }


def parse_junit_report(path: str | Path) -> dict[str, Any]:
    """Counts and per-case outcomes of a JUnit report.  Suite-level counts
    win over the case list when larger (a collection error is counted by the
    suite without a case); ``status`` is ``passed`` when nothing failed or
    errored, ``missing`` when the file does not exist."""
    p = Path(path)
    if not p.exists():
        return {"path": str(p), "status": "missing", **_EMPTY_COUNTS, "cases": []}
    root = ET.parse(p).getroot()
    suites = [root] if root.tag == "testsuite" else root.findall("testsuite")
    cases = [_case(c) for c in root.iter("testcase")]

    def count(attr: str, outcome: str) -> int:
        return max(sum(_int(s.get(attr)) for s in suites),
                   sum(1 for c in cases if c["outcome"] == outcome))

    tests = max(sum(_int(s.get("tests")) for s in suites), len(cases))
    failed, errors, skipped = count("failures", "failed"), count("errors", "error"), count(
        "skipped", "skipped")
    return {
        "path": str(p),
        "status": "passed" if failed == 0 and errors == 0 else "failed",
        "tests": tests,
        "passed": max(tests - failed - errors - skipped, 0),
        "failed": failed,
        "errors": errors,
        "skipped": skipped,
        "cases": cases,
    }


def load_benchmark_report(path: str | Path) -> dict[str, Any]:
    """The JSON written by ``BenchmarkReport.dump_json`` plus ``path`` and
    ``status`` (``present`` / ``missing``)."""
    p = Path(path)
    if not p.exists():
        return {"path": str(p), "status": "missing", "schema_version": 1, "records": []}
    data = json.loads(p.read_text(encoding="utf-8"))
    data["path"] = str(p)
    data["status"] = "present"
    return data
