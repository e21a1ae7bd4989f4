"""``tileops-report``: run an operator's correctness tests, then (only if they
pass) its benchmarks, and write ``run.json`` / ``report.md`` / ``report.html``.

Layout of the reference's package (examples/TileOPs/tileops/reporting/):
``collector`` (JUnit XML, benchmark JSON), ``analyzer`` (the run schema),
``report`` (renderers), ``setup_info`` (environment), ``runner`` (the
stage-gated pytest driver) and ``cli``.
"""

from tileops.reporting.analyzer import analyze_run
from tileops.reporting.collector import load_benchmark_report, parse_junit_report
from tileops.reporting.report import render_html, render_markdown, write_reports

__all__ = [
    "analyze_run",
    "load_benchmark_report",
    "parse_junit_report",
    "render_html",
    "render_markdown",
    "write_reports",
]
