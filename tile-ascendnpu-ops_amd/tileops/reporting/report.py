"""Markdown and HTML views of a run document, plus the writer of all three
files (``run.json``, ``report.md``, ``report.html``).

Views of the reference's renderer (examples/TileOPs/tileops/reporting/report.py:278-717):
setup tables, a results overview, per-operator analysis (pass rate, mean of
the per-case max abs error, roofline ratio range), per-case performance
rows, warnings and failed cases.  The HTML view is self-contained (inline
CSS, no template file, no script).
"""

from __future__ import annotations

import html
import json
from copy import deepcopy
from pathlib import Path
from typing import Any

from tileops.reporting.session_timing import format_duration

_SHAPE_EXCLUDE = {"dtype", "dtypes", "op_params", "case_id", "label"}


def _fmt(value: Any, digits: int = 4) -> str:
    if value is None:
        return "N/A"
    if isinstance(value, float):
        return f"{value:.{digits}f}"
    return str(value)


def _rate(value: Any) -> str:
    return f"{value:.1%}" if isinstance(value, (int, float)) else "N/A"


def _sci(value: Any) -> str:
    return f"{value:.2e}" if isinstance(value, (int, float)) else "N/A"


def _range(value: dict[str, Any] | None, suffix: str = "%", digits: int = 2) -> str:
    if not value:
        return "N/A"
    lo, hi = value.get("min"), value.get("max")
    if not isinstance(lo, (int, float)) or not isinstance(hi, (int, float)):
        return "N/A"
    if lo == hi:
        return f"{lo:.{digits}f}{suffix}"
    return f"{lo:.{digits}f}{suffix} – {hi:.{digits}f}{suffix}"


def _display(value: Any) -> str:
    if isinstance(value, (dict, list, tuple)):
        return json.dumps(value, ensure_ascii=False, separators=(", ", ": "))
    return "N/A" if value is None else str(value)


def _shape(params: dict[str, Any]) -> str:
    items = [(k, v) for k, v in params.items()
             if k == "shape" or k.endswith("_shape") or k.endswith("_shapes")]
    if len(items) == 1 and items[0][0] == "shape":
        return _display(items[0][1])
    if items:
        return "; ".join(f"{k}={_display(v)}" for k, v in items)
    rest = {k: v for k, v in params.items() if k not in _SHAPE_EXCLUDE and not k.endswith("_dtype")}
    return _display(rest) if rest else "N/A"


def _dtype(params: dict[str, Any]) -> str:
    items = [(k, v) for k, v in params.items() if k in {"dtype", "dtypes"} or k.endswith("_dtype")]
    if len(items) == 1:
        return _display(items[0][1])
    return "; ".join(f"{k}={_display(v)}" for k, v in items) or "N/A"


def _label(case: dict[str, Any]) -> str:
    label = case.get("label") or (case.get("params") or {}).get("label")
    return str(label) if label not in (None, "") else _shape(case.get("params") or {})


def _kernels(case: dict[str, Any]) -> str:
    names = case.get("kernels") or []
    return ", ".join(n.split("(")[0][:60] for n in names) if names else "N/A"


def _cell(value: Any) -> str:
    return str(value).replace("|", "\\|").replace("\n", " ")


def _normalize(run: dict[str, Any]) -> dict[str, Any]:
    """Fill what an older run document lacks (operators, summary, setup) so
    both schema versions render."""
    run = deepcopy(run)
    perf = (run.get("performance") or {}).get("cases", [])
    run.setdefault("performance", {"cases": perf})
    if not run.get("operators"):
        names = sorted({c.get("operator") for c in perf if c.get("operator")}) or [
            run.get("operator", "unknown")]
        corr = run.get("correctness") or {}
        ops = []
        for name in names:
            mine = [c for c in perf if c.get("operator") == name]
            ratios = [c["roofline_utilization_percent"] for c in mine
                      if isinstance(c.get("roofline_utilization_percent"), (int, float))]
            total = int(corr.get("tests", 0) or 0) if len(names) == 1 else 0
            passed = int(corr.get("passed", 0) or 0) if len(names) == 1 else 0
            ops.append({"operator": name, "cases": total, "passed": passed,
                        "failed": total - passed, "pass_rate": passed / total if total else None,
                        "avg_max_abs_err": None, "performance_cases": len(mine),
                        "ratio_range": {"min": min(ratios), "max": max(ratios)} if ratios else None})
        run["operators"] = ops
    summary = run.setdefault("summary", {})
    if "total_cases" not in summary:
        corr = run.get("correctness") or {}
        total = int(corr.get("tests", 0) or 0)
        passed = int(corr.get("passed", 0) or 0)
        summary.update({"total_cases": total, "passed_cases": passed,
                        "failed_cases": int(corr.get("failed", 0) or 0) + int(corr.get("errors", 0) or 0),
                        "pass_rate": passed / total if total else None,
                        "operator_count": len(run["operators"])})
    run.setdefault("setup", {})
    run.setdefault("warnings", [])
    return run


def _failed_cases(run: dict[str, Any]) -> list[tuple[str, dict]]:
    return [(stage, c) for stage, rep in (("Correctness", run.get("correctness") or {}),
                                          ("Benchmark", run.get("benchmark_tests") or {}))
            for c in rep.get("cases", []) if c.get("outcome") in {"failed", "error"}]


_PERF_HEAD = ("Label", "Latency (us)", "Ratio (%)", "AI (Ops/Byte)", "Bound", "Shape / Parameters",
              "DType", "Mode", "Kernels", "Bandwidth (TB/s)", "Perf (TOps/s)")
# with rocprofv3 counters (tileops-report run --with-counters)
_COUNTER_HEAD = ("HBM (TB/s, counters)", "HBM bytes / roofline bytes", "MFMA busy (%)")


def _has_counters(cases: list[dict[str, Any]]) -> bool:
    return any(c.get("hbm_bytes_measured") is not None for c in cases)


def _perf_row(case: dict[str, Any], counters: bool = False) -> list[str]:
    p = case.get("params") or {}
    row = [_label(case), _fmt(case.get("latency_us")), _fmt(case.get("roofline_utilization_percent"), 2),
           _fmt(case.get("arithmetic_intensity_ops_per_byte")), case.get("bound") or "?",
           _shape(p), _dtype(p), case.get("prof_mode") or "N/A", _kernels(case),
           _fmt(case.get("bandwidth_tb_s")), _fmt(case.get("performance_tops"))]
    if counters:
        bw, lat = case.get("bandwidth_tb_s"), case.get("latency_us")
        roof = bw * lat * 1e6 if isinstance(bw, (int, float)) and isinstance(lat, (int, float)) else None
        meas = case.get("hbm_bytes_measured")
        ratio = meas / roof if meas is not None and roof else None
        row += [_fmt(case.get("hbm_tb_s_measured")), _fmt(ratio, 3), _fmt(case.get("mfma_busy_percent"), 1)]
    return row


def _timing(run: dict[str, Any]) -> list[tuple[str, dict]]:
    """(operator, record) pairs of an enabled session-timing section."""
    st = run.get("session_timing") or {}
    if not st.get("enabled"):
        return []
    return [(name, rec or {}) for name, rec in (st.get("operators") or {}).items()]


def _timing_breakdown(rec: dict[str, Any]) -> str:
    if rec.get("status") != "available":
        return f"Timing data unavailable: {rec.get('reason') or rec.get('status', 'unknown')}"
    parts = []
    for b in rec.get("breakdown") or []:
        ratio = b.get("ratio_percent")
        pct = f" ({ratio:.2f}%)" if isinstance(ratio, (int, float)) else ""
        parts.append(f"{b.get('name')}: {format_duration(b.get('duration_s'))}{pct}")
    return "; ".join(parts) or "-"


def render_markdown(run: dict[str, Any]) -> str:
    run = _normalize(run)
    s = run["summary"]
    lines = [f"# TileOPs Evaluation Report: {run.get('operator', 'unknown')}", ""]
    for title, key in (("Metadata", "metadata"), ("Environment", "environment")):
        block = (run.get("setup") or {}).get(key) or {}
        if block:
            lines += [f"## {title}", "", "| Field | Value |", "|---|---|"]
            lines += [f"| {k} | {_cell(_display(v))} |" for k, v in block.items()]
            lines.append("")
    lines += ["## Results Overview", "", "| Pass Rate | Operators | Total Cases | Failed Cases |",
              "|---:|---:|---:|---:|",
              f"| {_rate(s.get('pass_rate'))} | {s.get('operator_count', 0)} | "
              f"{s.get('total_cases', 0)} | {s.get('failed_cases', 0)} |", "",
              "## Operator Analysis", "",
              "| Operator | Correctness | Avg Max Abs Error | Performance Shapes | Ratio Range |",
              "|---|---:|---:|---:|---:|"]
    for op in run["operators"]:
        lines.append(f"| {_cell(op.get('operator'))} | {_rate(op.get('pass_rate'))} "
                     f"({op.get('passed', 0)}/{op.get('cases', 0)}) | {_sci(op.get('avg_max_abs_err'))} | "
                     f"{op.get('performance_cases', 0)} | {_range(op.get('ratio_range'))} |")
    lines += ["", "> Correctness: pass rate (passed / total cases).  Ratio: roofline floor time "
              "over measured latency per shape, against MI355X peaks (HBM 8 TB/s; MFMA "
              "2516.6 TFLOP/s fp16/bf16; 157.3 TFLOP/s fp32).", "", "## Operator Details", ""]
    perf = run["performance"].get("cases", [])
    counters = _has_counters(perf)
    head = _PERF_HEAD + (_COUNTER_HEAD if counters else ())
    if counters:
        lines += ["> Counters (rocprofv3): HBM bytes per call from FETCH_SIZE / WRITE_SIZE scaled "
                  "by a device-copy calibration, and their ratio to the roofline bytes; MFMA busy "
                  "= SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs x GRBM_GUI_ACTIVE / 8).", ""]
    for op in run["operators"]:
        name = op.get("operator")
        cases = [c for c in perf if c.get("operator") == name]
        lines += [f"### {name}", "", "| " + " | ".join(head) + " |",
                  "|---|---:|---:|---:|:---:|---|---|---|---|---:|---:|" + ("---:|" * 3 if counters else "")]
        lines += ["| " + " | ".join(_cell(x) for x in _perf_row(c, counters)) + " |" for c in cases]
        if not cases:
            lines.append("| - | No performance records |" + " - |" * (len(head) - 2))
        lines.append("")
    timing = _timing(run)
    if timing:
        lines += ["## Session Timing", "", "| Operator | Total Time | Breakdown |", "|---|---:|---|"]
        lines += [f"| {_cell(name)} | {format_duration(rec.get('total_duration_s'))} | "
                  f"{_cell(_timing_breakdown(rec))} |" for name, rec in timing]
        lines.append("")
    if run["warnings"]:
        lines += ["## Warnings", "", *(f"- {w}" for w in run["warnings"]), ""]
    failed = _failed_cases(run)
    if failed:
        lines += ["## Failed Cases", "", "| Stage | Test | Outcome | Message |", "|---|---|---|---|"]
        lines += [f"| {st} | {_cell(c.get('nodeid'))} | {c.get('outcome')} | {_cell(c.get('message') or '')} |"
                  for st, c in failed]
        lines.append("")
    return "\n".join(lines)


_CSS = """
body{font-family:system-ui,sans-serif;margin:2em;color:#222}
table{border-collapse:collapse;margin:0.5em 0 1.5em}
th,td{border:1px solid #ccc;padding:4px 8px;font-size:13px}
th{background:#f3f3f3}
td.num{text-align:right;font-variant-numeric:tabular-nums}
.passed{color:#17803d}.failed{color:#b42318}.partial{color:#b54708}
.hi{background:#e7f6ec}.mid{background:#fff7e0}.lo{background:#fdecea}
"""


def _table(head: list[str] | tuple[str, ...], rows: list[list[str]], numeric: set[int] = frozenset()) -> str:
    th = "".join(f"<th>{html.escape(h)}</th>" for h in head)
    body = []
    for r in rows:
        cells = []
        for i, v in enumerate(r):
            cls = ' class="num"' if i in numeric else ""
            cells.append(f"<td{cls}>{html.escape(str(v))}</td>")
        body.append("<tr>" + "".join(cells) + "</tr>")
    return f"<table><thead><tr>{th}</tr></thead><tbody>{''.join(body)}</tbody></table>"


def render_html(run: dict[str, Any]) -> str:
    run = _normalize(run)
    s = run["summary"]
    status = str(run.get("status", "unknown"))
    parts = [f"<h1>TileOPs Evaluation Report: {html.escape(str(run.get('operator', 'unknown')))}</h1>",
             f'<p>Status: <b class="{html.escape(status)}">{html.escape(status)}</b></p>']
    for title, key in (("Metadata", "metadata"), ("Environment", "environment")):
        block = (run.get("setup") or {}).get(key) or {}
        if block:
            parts.append(f"<h2>{title}</h2>")
            parts.append(_table(["Field", "Value"], [[k, _display(v)] for k, v in block.items()]))
    parts.append("<h2>Results Overview</h2>")
    parts.append(_table(["Pass Rate", "Operators", "Total Cases", "Failed Cases"],
                        [[_rate(s.get("pass_rate")), s.get("operator_count", 0), s.get("total_cases", 0),
                          s.get("failed_cases", 0)]], {0, 1, 2, 3}))
    parts.append("<h2>Operator Analysis</h2>")
    parts.append(_table(["Operator", "Correctness", "Avg Max Abs Error", "Performance Shapes", "Ratio Range"],
                        [[op.get("operator"), f"{_rate(op.get('pass_rate'))} ({op.get('passed', 0)}/"
                          f"{op.get('cases', 0)})", _sci(op.get("avg_max_abs_err")),
                          op.get("performance_cases", 0), _range(op.get("ratio_range"))]
                         for op in run["operators"]], {1, 2, 3, 4}))
    parts.append("<h2>Operator Details</h2>")
    perf = run["performance"].get("cases", [])
    counters = _has_counters(perf)
    head = list(_PERF_HEAD + (_COUNTER_HEAD if counters else ()))
    numeric = {1, 2, 3, 9, 10} | ({11, 12, 13} if counters else set())
    for op in run["operators"]:
        cases = [c for c in perf if c.get("operator") == op.get("operator")]
        parts.append(f"<h3>{html.escape(str(op.get('operator')))}</h3>")
        parts.append(_table(head, [_perf_row(c, counters) for c in cases], numeric)
                     if cases else "<p>No performance records.</p>")
    timing = _timing(run)
    if timing:
        parts.append("<h2>Session Timing / Session 耗时</h2>")
        parts.append(_table(["Operator", "Total Time / 总时间", "Breakdown"],
                            [[name, format_duration(rec.get("total_duration_s")),
                              _timing_breakdown(rec)] for name, rec in timing], {1}))
    if run["warnings"]:
        parts.append("<h2>Warnings</h2><ul>" + "".join(
            f"<li>{html.escape(str(w))}</li>" for w in run["warnings"]) + "</ul>")
    failed = _failed_cases(run)
    if failed:
        parts.append("<h2>Failed Cases</h2>")
        parts.append(_table(["Stage", "Test", "Outcome", "Message"],
                            [[st, c.get("nodeid"), c.get("outcome"), c.get("message") or ""]
                             for st, c in failed]))
    title = html.escape(f"TileOPs report: {run.get('operator', 'unknown')}")
    return (f"<!DOCTYPE html><html><head><meta charset=\"utf-8\"><title>{title}</title>"
            f"<style>{_CSS}</style></head><body>{''.join(parts)}</body></html>\n")


def write_reports(run: dict[str, Any], output_dir: str | Path) -> dict[str, Path]:
    """Write ``run.json``, ``report.md`` and ``report.html`` into ``output_dir``."""
    root = Path(output_dir)
    root.mkdir(parents=True, exist_ok=True)
    paths = {"json": root / "run.json", "markdown": root / "report.md", "html": root / "report.html"}
    paths["json"].write_text(json.dumps(run, indent=2, ensure_ascii=False), encoding="utf-8")
    paths["markdown"].write_text(render_markdown(run), encoding="utf-8")
    paths["html"].write_text(render_html(run), encoding="utf-8")
    return paths
