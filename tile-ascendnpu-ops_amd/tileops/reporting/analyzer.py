"""Turn correctness (JUnit) and benchmark records into the run document.

Schema of the reference's analyzer (examples/TileOPs/tileops/reporting/analyzer.py:234-321,
``schema_version`` 2): run ``status`` is ``failed`` when correctness failed,
``passed`` when the benchmark stage also produced valid records, else
``partial``.  Benchmark records are grouped per (operator, case); only
``tileops*``-tagged records count, smoke-labelled records never reach the
performance tables, and a record whose timing fell back from the requested
profiler, or whose kernel filter matched nothing, is flagged.
"""

from __future__ import annotations

import math
import re
from collections import defaultdict
from pathlib import PurePosixPath
from typing import Any

_SMOKE = re.compile(r"(?:^|[^a-z0-9])smoke(?:$|[^a-z0-9])", re.IGNORECASE)


def _profile_validity(result: dict[str, Any]) -> tuple[bool, str | None]:
    if result.get("prof_mode") != "rocprof":
        return True, None
    meta = result.get("rocprof") or {}
    if meta.get("kernel_name_requested") and not meta.get("kernel_name_resolved"):
        return False, f"kernel filter {meta['kernel_name_requested']!r} matched no kernel"
    if not meta.get("kernels"):
        return False, "no kernel dispatch matched the filter"
    return True, None


def _is_smoke_record(record: dict[str, Any]) -> bool:
    params = record.get("params") or {}
    return any(isinstance(v, str) and _SMOKE.search(v)
               for v in (record.get("label"), params.get("label")))


def _analyze_performance(benchmark: dict[str, Any]) -> tuple[list[dict], dict, list[str]]:
    requested = benchmark.get("profiling_mode_requested")
    groups: dict[tuple[str, str], list[dict]] = defaultdict(list)
    for rec in benchmark.get("records", []):
        if str(rec.get("tag", "")).startswith("tileops"):
            groups[(rec.get("operator", "unknown"), rec.get("case_id", "unknown"))].append(rec)
    cases, warnings = [], []
    fallback = invalid = 0
    for (operator, case_id), recs in groups.items():
        if any(_is_smoke_record(r) for r in recs):
            continue
        rec = recs[0]
        result = rec.get("result", {})
        mode = result.get("prof_mode")
        valid, reason = _profile_validity(result)
        if not valid:
            invalid += 1
            warnings.append(f"{operator}/{case_id}: invalid tileops profile: {reason}")
        if requested == "rocprof" and mode != "rocprof":
            fallback += 1
            why = result.get("rocprof_fallback")
            warnings.append(f"{operator}/{case_id}: requested rocprof but recorded {mode or 'unknown'}"
                            + (f" ({why})" if why else ""))
        ctr_err = (result.get("rocprof") or {}).get("counters_error")
        if ctr_err:
            warnings.append(f"{operator}/{case_id}: counter collection failed ({ctr_err})")
        meta = result.get("rocprof") or None
        cases.append({
            "operator": operator,
            "case_id": case_id,
            "label": rec.get("label") or rec.get("params", {}).get("label"),
            "params": rec.get("params", {}),
            "config": rec.get("config"),
            "tag": rec.get("tag", "tileops"),
            "latency_us": result.get("latency_us"),
            "prof_mode": mode,
            "profiler_valid": valid,
            "invalid_reason": reason,
            "roofline_utilization_percent": result.get("Ratio(%)"),
            "bandwidth_tb_s": result.get("Bandwidth(TB/s)", result.get("bandwidth_tbs")),
            "arithmetic_intensity_ops_per_byte": result.get("AI(Ops/Byte)"),
            "performance_tops": result.get("Perf(TOps/s)", result.get("tflops")),
            "computility_tops": result.get("Computility(TOPs/s)"),
            "bound": result.get("bound"),
            "hbm_bytes_measured": result.get("HBM bytes (counters)"),
            "hbm_tb_s_measured": result.get("HBM(TB/s, counters)"),
            "mfma_busy_percent": result.get("MFMA busy(%)"),
            "kernels": [k.get("name") for k in (meta or {}).get("kernels", [])] or None,
            "rocprof": meta,
        })
    summary = {
        "case_count": len(cases),
        "rocprof_case_count": sum(1 for c in cases if c["prof_mode"] == "rocprof"),
        "profiler_fallback_count": fallback,
        "invalid_profile_count": invalid,
    }
    return cases, summary, warnings


def _test_key(path: str | None) -> str:
    return PurePosixPath(path.replace("\\", "/")).stem.lower() if path else ""


def _keyword_match(expr: str, hay: str) -> bool:
    """A manifest ``test_keyword`` (pytest ``-k`` terms joined by ``or``)
    against a lower-cased case name."""
    terms = [t.strip().lower() for t in str(expr).split(" or ") if t.strip()]
    return any(t in hay for t in terms)


def _case_operator(case: dict[str, Any], catalog: list[dict[str, Any]],
                   default: str | None) -> str | None:
    """The op a JUnit case belongs to: its ``op`` property, else the one
    manifest op whose test file names it; when several ops share that file,
    the one whose class name appears in the case id, else the one whose
    ``test_keyword`` matches it; else ``default``."""
    declared = (case.get("properties") or {}).get("op")
    if declared:
        return str(declared)
    hay = f"{case.get('classname', '')} {case.get('nodeid', '')} {case.get('name', '')}".lower()
    hits = [e for e in catalog if _test_key(e.get("test")) and _test_key(e.get("test")) in hay]
    names = {e.get("name") for e in hits}
    if len(names) == 1:
        return hits[0].get("name")
    if len(names) > 1:
        by_class = {n for n in names if n and n.lower() in hay}
        if len(by_class) == 1:
            return by_class.pop()
        by_kw = {e.get("name") for e in hits if e.get("test_keyword") and _keyword_match(e["test_keyword"], hay)}
        if len(by_kw) == 1:
            return by_kw.pop()
    return default


def _num_prop(case: dict[str, Any], name: str) -> float | None:
    try:
        v = float((case.get("properties") or {}).get(name))
    except (TypeError, ValueError):
        return None
    return v if math.isfinite(v) else None


def _analyze_operators(*, requested_operator: str, correctness: dict[str, Any],
                       perf_cases: list[dict[str, Any]],
                       operator_catalog: list[dict[str, Any]]) -> list[dict[str, Any]]:
    if requested_operator == "all":
        names = [str(e["name"]) for e in operator_catalog if e.get("name")]
        seen = {str(c.get("operator")) for c in perf_cases if c.get("operator")}
        seen |= {str((c.get("properties") or {}).get("op")) for c in correctness.get("cases", [])
                 if (c.get("properties") or {}).get("op")}
        names.extend(sorted(seen.difference(names)))
    else:
        names = [requested_operator]
    by_name = {str(e.get("name")): e for e in operator_catalog}
    per_op: dict[str, list[dict]] = defaultdict(list)
    default = names[0] if len(names) == 1 else None
    for case in correctness.get("cases", []):
        op = _case_operator(case, operator_catalog, default)
        if op:
            per_op[op].append(case)
    out = []
    for name in names:
        mine = per_op.get(name, [])
        if len(names) == 1 and not mine and not correctness.get("cases"):
            total = int(correctness.get("tests", 0) or 0)
            passed = int(correctness.get("passed", 0) or 0)
            failed = int(correctness.get("failed", 0) or 0) + int(correctness.get("errors", 0) or 0)
        else:
            total = len(mine)
            passed = sum(1 for c in mine if c.get("outcome") == "passed")
            failed = sum(1 for c in mine if c.get("outcome") in {"failed", "error"})
        op_perf = [c for c in perf_cases if c.get("operator") == name]
        ratios = [float(c["roofline_utilization_percent"]) for c in op_perf
                  if isinstance(c.get("roofline_utilization_percent"), (int, float))]
        errs = [v for c in mine if (v := _num_prop(c, "max_abs_err")) is not None]
        out.append({
            "operator": name,
            "family": by_name.get(name, {}).get("family"),
            "cases": total,
            "passed": passed,
            "failed": failed,
            "pass_rate": passed / total if total else None,
            "avg_max_abs_err": sum(errs) / len(errs) if errs else None,
            "max_abs_err": max(errs) if errs else None,
            "performance_cases": len(op_perf),
            "ratio_range": {"min": min(ratios), "max": max(ratios)} if ratios else None,
        })
    return out


def analyze_run(
    *,
    operator: str,
    correctness: dict[str, Any],
    correctness_exit_code: int,
    benchmark: dict[str, Any] | None = None,
    benchmark_exit_code: int | None = None,
    benchmark_tests: dict[str, Any] | None = None,
    metadata: dict[str, Any] | None = None,
    setup: dict[str, Any] | None = None,
    operator_catalog: list[dict[str, Any]] | None = None,
) -> dict[str, Any]:
    """The canonical run document every renderer consumes."""
    benchmark = benchmark or {"records": [], "status": "skipped"}
    benchmark_tests = benchmark_tests or {"status": "skipped", "tests": 0, "passed": 0,
                                          "failed": 0, "errors": 0, "skipped": 0, "cases": []}
    perf_cases, perf_summary, warnings = _analyze_performance(benchmark)
    operators = _analyze_operators(requested_operator=operator, correctness=correctness,
                                   perf_cases=perf_cases, operator_catalog=operator_catalog or [])
    correct_ok = correctness_exit_code == 0 and correctness.get("status") == "passed"
    bench_requested = benchmark_exit_code is not None
    bench_failed = int(benchmark_tests.get("failed", 0) or 0) + int(benchmark_tests.get("errors", 0) or 0)
    bench_ok = (bench_requested and benchmark_exit_code == 0 and benchmark.get("status") == "present"
                and bool(perf_cases) and perf_summary["profiler_fallback_count"] == 0
                and perf_summary["invalid_profile_count"] == 0 and bench_failed == 0)
    if correct_ok and bench_requested and not bench_ok:
        warnings.append("correctness passed, but the benchmark stage did not produce valid records")
    if bench_failed:
        warnings.append(f"benchmark pytest reported {bench_failed} failed/error cases")
    total = int(correctness.get("tests", 0) or 0)
    passed = int(correctness.get("passed", 0) or 0)
    failed = int(correctness.get("failed", 0) or 0) + int(correctness.get("errors", 0) or 0)
    return {
        "schema_version": 2,
        "operator": operator,
        "status": "failed" if not correct_ok else "passed" if bench_ok else "partial",
        "metadata": metadata or {},
        "setup": setup or {},
        "summary": {
            "correctness_passed": correct_ok,
            "correctness_tests": correctness.get("tests", 0),
            "correctness_failed": correctness.get("failed", 0) + correctness.get("errors", 0),
            "operator_count": len(operators),
            "total_cases": total,
            "passed_cases": passed,
            "failed_cases": failed,
            "pass_rate": passed / total if total else None,
            "benchmark_requested": bench_requested,
            "benchmark_passed": bench_ok,
            "benchmark_tests": benchmark_tests.get("tests", 0),
            "benchmark_failed": bench_failed,
            **perf_summary,
        },
        "correctness": correctness,
        "benchmark_tests": benchmark_tests,
        "performance": {
            "source": benchmark.get("path"),
            "requested_prof_mode": benchmark.get("profiling_mode_requested"),
            "cases": perf_cases,
        },
        "operators": operators,
        "warnings": warnings,
    }
