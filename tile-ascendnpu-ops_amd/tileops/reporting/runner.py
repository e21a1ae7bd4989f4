"""Stage-gated runner: correctness pytest first, benchmark pytest only if it
passed, then the run document and its reports in one directory.

Behaviour of the reference's runner (examples/TileOPs/tileops/reporting/runner.py:178-329):
targets resolve from the manifest's ``source.test`` / ``source.bench`` (or
explicit overrides; ``all`` runs the whole test and benchmark trees);
pytest-xdist is refused (workers would overwrite one another's benchmark
JSON); smoke cases are excluded from the benchmark stage; each stage runs in
a child ``python -m pytest`` with a JUnit report; ``latest.json`` points at
the newest run.  The manifest's ``source.test_keyword``, when present, is
passed to the correctness stage as ``-k``.  This process never touches the
GPU itself: only the pytest children do.
"""

from __future__ import annotations

import json
import os
import platform
import re
import shlex
import subprocess
import sys
from datetime import datetime
from pathlib import Path
from typing import Any

from tileops.manifest import load_manifest
from tileops.reporting.analyzer import analyze_run
from tileops.reporting.collector import load_benchmark_report, parse_junit_report
from tileops.reporting.report import write_reports
from tileops.reporting.session_timing import attach_session_timing
from tileops.reporting.setup_info import collect_setup_info

ALL_TESTS = "tests/ops"
ALL_BENCHMARKS = "tile-ascendnpu-ops_amd/benchmarks/ops"


def project_root() -> Path:
    """The repository root (holds ``tests/`` and the package directory)."""
    return Path(__file__).resolve().parents[3]


def list_operators() -> list[dict[str, Any]]:
    """Manifest operators with their family, status and declared sources."""
    out = []
    for name, entry in sorted(load_manifest().items()):
        src = entry.get("source") or {}
        out.append({
            "name": name,
            "family": entry.get("family"),
            "status": entry.get("status"),
            "test": src.get("test"),
            "test_keyword": src.get("test_keyword"),
            "benchmark": src.get("bench"),
            "kernel": src.get("kernel"),
        })
    return out


def resolve_operator(operator: str, *, test_file: str | None = None,
                     benchmark_file: str | None = None) -> tuple[str, str]:
    """``(test_target, benchmark_target)`` of ``operator``."""
    if operator == "all" and not test_file and not benchmark_file:
        return ALL_TESTS, ALL_BENCHMARKS
    src = (load_manifest().get(operator) or {}).get("source") or {}
    test = test_file or src.get("test")
    bench = benchmark_file or src.get("bench")
    if not test or not bench:
        raise ValueError(
            f"operator {operator!r} must declare source.test/source.bench in the manifest "
            "or receive --test-file and --benchmark-file"
        )
    return str(test), str(bench)


def _test_keyword(operator: str, test_file: str | None) -> str | None:
    if operator == "all" or test_file:
        return None
    return ((load_manifest().get(operator) or {}).get("source") or {}).get("test_keyword")


def _safe_name(value: str) -> str:
    return re.sub(r"[^A-Za-z0-9_.-]+", "_", value).strip("_") or "operator"


def _reject_xdist(pytest_args: list[str], pytest_addopts: str | None) -> None:
    """``ValueError`` for any pytest-xdist worker request (``-n N``,
    ``-nN``, ``--numprocesses[=]N`` with N other than 0)."""
    args = [*pytest_args, *shlex.split(pytest_addopts or "")]
    for i, a in enumerate(args):
        nxt = args[i + 1] if i + 1 < len(args) else ""
        if a in ("-n", "--numprocesses"):
            bad = nxt not in {"", "0"}
        elif a.startswith("--numprocesses="):
            bad = a != "--numprocesses=0"
        elif a.startswith("-n") and len(a) > 2:
            bad = a != "-n0"
        else:
            bad = False
        if bad:
            raise ValueError(
                "pytest-xdist is not supported by tileops-report: benchmark workers "
                "would overwrite benchmark.json. Run the report serially."
            )


def _exclude_smoke(pytest_args: list[str]) -> list[str]:
    """``pytest_args`` with every marker expression merged and ``not smoke``
    added: ``-m "(a) and (b) and not smoke"``."""
    rest, exprs = [], []
    i = 0
    while i < len(pytest_args):
        a = pytest_args[i]
        if a in ("-m", "--markexpr"):
            if i + 1 >= len(pytest_args):
                raise ValueError(f"{a} requires a marker expression")
            exprs.append(pytest_args[i + 1])
            i += 2
            continue
        if a.startswith("--markexpr=") or a.startswith("-m="):
            exprs.append(a.split("=", 1)[1])
        else:
            rest.append(a)
        i += 1
    joined = " and ".join(f"({e})" for e in exprs if e.strip())
    return [*rest, "-m", f"{joined} and not smoke" if joined else "not smoke"]


def _with_keyword(pytest_args: list[str], keyword: str | None) -> list[str]:
    if not keyword:
        return list(pytest_args)
    out, found = [], False
    i = 0
    while i < len(pytest_args):
        if pytest_args[i] == "-k" and i + 1 < len(pytest_args):
            out += ["-k", f"({pytest_args[i + 1]}) and ({keyword})"]
            found = True
            i += 2
            continue
        out.append(pytest_args[i])
        i += 1
    return out if found else [*out, "-k", keyword]


def _git_commit(root: Path) -> str | None:
    try:
        res = subprocess.run(["git", "rev-parse", "HEAD"], cwd=root, capture_output=True,
                             text=True, check=False, timeout=10)
    except (OSError, subprocess.SubprocessError):
        return None
    return res.stdout.strip() if res.returncode == 0 else None


def _run_pytest(*, root: Path, target: str, junit_path: Path, log_path: Path,
                env: dict[str, str], pytest_args: list[str],
                timeout: int | None) -> tuple[int, list[str]]:
    cmd = [sys.executable, "-m", "pytest", target, "-sv", f"--junitxml={junit_path}", *pytest_args]
    with log_path.open("w", encoding="utf-8") as log:
        log.write(f"command: {' '.join(cmd)}\n\n")
        log.flush()
        try:
            res = subprocess.run(cmd, cwd=root, env=env, stdout=log, stderr=subprocess.STDOUT,
                                 check=False, timeout=timeout)
            return res.returncode, cmd
        except subprocess.TimeoutExpired:
            log.write(f"\nERROR: pytest timed out after {timeout} seconds\n")
            return 124, cmd


def run_operator(
    operator: str,
    *,
    test_file: str | None = None,
    benchmark_file: str | None = None,
    prof_mode: str = "rocprof",
    kernel_name: str | None = None,
    reports_dir: str | Path = "reports/tileops",
    pytest_args: list[str] | None = None,
    timeout: int | None = None,
    root: str | Path | None = None,
    with_session_timing: bool = False,
    with_counters: bool = False,
) -> tuple[dict[str, Any], Path, int]:
    """Run one operator (or ``all``) and write its report directory.

    Returns ``(run, run_dir, exit_code)``; the exit code is 0 only when the
    run status is ``passed``."""
    repo = Path(root).resolve() if root else project_root()
    test_target, bench_target = resolve_operator(operator, test_file=test_file,
                                                 benchmark_file=benchmark_file)
    for target in (test_target, bench_target):
        if not (repo / target).exists():
            raise FileNotFoundError(f"pytest target does not exist: {repo / target}")
    args = list(pytest_args or [])
    env = dict(os.environ)
    _reject_xdist(args, env.get("PYTEST_ADDOPTS"))

    stamp = datetime.now().strftime("%Y%m%d_%H%M%S_%f")
    run_dir = (repo / reports_dir / f"{stamp}_{_safe_name(operator)}").resolve()
    pytest_dir = run_dir / "pytest"
    artifact_dir = run_dir / "artifacts" / "rocprof"
    pytest_dir.mkdir(parents=True, exist_ok=True)
    artifact_dir.mkdir(parents=True, exist_ok=True)

    print(f"[tileops-report] correctness: {test_target}", flush=True)
    corr_xml = pytest_dir / "correctness.xml"
    corr_code, corr_cmd = _run_pytest(
        root=repo, target=test_target, junit_path=corr_xml, log_path=pytest_dir / "correctness.log",
        env=env, pytest_args=_with_keyword(args, _test_keyword(operator, test_file)), timeout=timeout)
    correctness = parse_junit_report(corr_xml)

    bench_code: int | None = None
    bench_cmd: list[str] | None = None
    benchmark: dict[str, Any] = {"status": "skipped", "records": []}
    bench_tests: dict[str, Any] = {"status": "skipped", "tests": 0, "passed": 0, "failed": 0,
                                   "errors": 0, "skipped": 0, "cases": []}
    if corr_code == 0 and correctness.get("status") == "passed":
        benv = dict(env)
        benv.update({
            "TILEOPS_PROF_MODE": prof_mode,
            "TILEOPS_ROCPROF_ARTIFACT_ROOT": str(artifact_dir),
            "TILEOPS_BENCHMARK_REPORT_PATH": str(run_dir / "benchmark.md"),
        })
        if kernel_name:
            benv["TILEOPS_ROCPROF_KERNEL_NAME"] = kernel_name
        else:
            benv.pop("TILEOPS_ROCPROF_KERNEL_NAME", None)
        if with_counters and prof_mode == "rocprof":
            benv["TILEOPS_ROCPROF_COUNTERS"] = "1"
        else:
            benv.pop("TILEOPS_ROCPROF_COUNTERS", None)
        print(f"[tileops-report] benchmark: {bench_target} ({prof_mode})", flush=True)
        bench_xml = pytest_dir / "benchmark.xml"
        bench_code, bench_cmd = _run_pytest(
            root=repo, target=bench_target, junit_path=bench_xml,
            log_path=pytest_dir / "benchmark.log", env=benv, pytest_args=_exclude_smoke(args),
            timeout=timeout)
        bench_tests = parse_junit_report(bench_xml)
        benchmark = load_benchmark_report(run_dir / "benchmark.json")
    else:
        print("[tileops-report] benchmark skipped because correctness did not pass", flush=True)

    generated_at = datetime.now().astimezone().isoformat()
    commit = _git_commit(repo)
    metadata = {
        "run_id": run_dir.name,
        "generated_at": generated_at,
        "project_root": str(repo),
        "git_commit": commit,
        "python": sys.version.split()[0],
        "platform": platform.platform(),
        "test_file": test_target,
        "benchmark_file": bench_target,
        "prof_mode_requested": prof_mode,
        "kernel_name_requested": kernel_name,
        "commands": {"correctness": corr_cmd, "benchmark": bench_cmd},
        "exit_codes": {"correctness": corr_code, "benchmark": bench_code},
    }
    catalog = list_operators()
    setup = collect_setup_info(scope=operator, run_id=run_dir.name, generated_at=generated_at,
                               profiler=prof_mode, git_commit=commit, test_target=test_target,
                               benchmark_target=bench_target)
    run = analyze_run(operator=operator, correctness=correctness, correctness_exit_code=corr_code,
                      benchmark=benchmark, benchmark_exit_code=bench_code,
                      benchmark_tests=bench_tests, metadata=metadata, setup=setup,
                      operator_catalog=catalog)
    attach_session_timing(run, root=Path(__file__).resolve().parents[2],
                          operator_catalog=catalog, enabled=with_session_timing)
    write_reports(run, run_dir)
    (run_dir.parent / "latest.json").write_text(
        json.dumps({"run_id": run_dir.name, "run_json": str(run_dir / "run.json")}, indent=2),
        encoding="utf-8")
    return run, run_dir, 0 if run["status"] == "passed" else 1
