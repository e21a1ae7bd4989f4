"""``tileops-report`` command line: ``list``, ``run``, ``render``.

Commands and options of the reference's CLI
(examples/TileOPs/tileops/reporting/cli.py:14-97), with the profiler
choices ``rocprof`` (default) and ``events``.  Run as
``python -m tileops.reporting.cli ...``.
"""

from __future__ import annotations

import argparse
import json
from pathlib import Path

from tileops.reporting.report import write_reports
from tileops.reporting.runner import list_operators, run_operator
from tileops.reporting.session_timing import attach_session_timing


def _parser() -> argparse.ArgumentParser:
    ap = argparse.ArgumentParser(
        prog="tileops-report",
        description="Run the TileOPs pytest gates and generate structured reports.")
    sub = ap.add_subparsers(dest="command", required=True)
    sub.add_parser("list", help="list operators declared in the manifest")
    run = sub.add_parser("run", help="run correctness, then benchmark and report")
    which = run.add_mutually_exclusive_group(required=True)
    which.add_argument("--op", help="manifest operator name")
    which.add_argument("--all", action="store_true",
                       help="run pytest tests/ops followed by the benchmark tree")
    run.add_argument("--test-file", help="override manifest source.test")
    run.add_argument("--benchmark-file", help="override manifest source.bench")
    run.add_argument("--prof-mode", choices=("rocprof", "events"), default="rocprof")
    run.add_argument("--kernel-name", help="kernel-name regex for rocprof (TILEOPS_ROCPROF_KERNEL_NAME)")
    run.add_argument("--reports-dir", default="reports/tileops")
    run.add_argument("--timeout", type=int, help="timeout in seconds for each pytest stage")
    run.add_argument("--pytest-arg", action="append", default=[],
                     help="additional pytest argument; repeat for several")
    run.add_argument("--with-counters", action="store_true",
                     help="rocprof mode: also collect HBM bytes (FETCH_SIZE / WRITE_SIZE) and "
                          "MFMA busy per case (three more profiled runs per case)")
    render = sub.add_parser("render", help="regenerate Markdown/HTML from run.json")
    render.add_argument("run_json")
    render.add_argument("--output-dir")
    for p in (run, render):
        p.add_argument("--with-session-timing", action="store_true",
                       help="add the per-operator SESSION_TIMING_ANALYSIS.md totals")
    return ap


def _package_root() -> Path:
    return Path(__file__).resolve().parents[2]


def main(argv: list[str] | None = None) -> int:
    args = _parser().parse_args(argv)
    if args.command == "list":
        for op in list_operators():
            print(f"{op['name']:<28} family={op['family'] or '-':<17} "
                  f"test={op['test'] or '-'} bench={op['benchmark'] or '-'}")
        return 0
    if args.command == "render":
        src = Path(args.run_json).resolve()
        run = json.loads(src.read_text(encoding="utf-8"))
        attach_session_timing(run, root=_package_root(), operator_catalog=list_operators(),
                              enabled=args.with_session_timing)
        paths = write_reports(run, Path(args.output_dir).resolve() if args.output_dir else src.parent)
        print(f"Reports written to {paths['markdown']} and {paths['html']}")
        return 0
    run, run_dir, code = run_operator(
        "all" if args.all else args.op, test_file=args.test_file,
        benchmark_file=args.benchmark_file, prof_mode=args.prof_mode,
        kernel_name=args.kernel_name, reports_dir=args.reports_dir,
        pytest_args=args.pytest_arg, timeout=args.timeout,
        with_session_timing=args.with_session_timing, with_counters=args.with_counters)
    print(f"[tileops-report] status={run['status']} report={run_dir / 'report.md'}")
    return code


if __name__ == "__main__":
    raise SystemExit(main())
