"""CPU tests of the report harness: JUnit / benchmark collectors, the run
analyzer, the renderers, the stage-gated runner (pytest stages faked), the
CLI, the benchmark report and the rocprof helpers.

Scenarios follow the reference's harness tests
(examples/TileOPs/tests/reporting/test_reporting.py:14-245, 389-659); the
fixtures are written here.
"""

import json
from pathlib import Path

import pytest
import torch

from tileops.benchmark import benchmark_base as bb
from tileops.benchmark import rocprof as rp
from tileops.reporting import analyzer, cli, runner
from tileops.reporting.collector import load_benchmark_report, parse_junit_report
from tileops.reporting.report import render_html, render_markdown, write_reports

JUNIT_OK = """<?xml version="1.0" encoding="utf-8"?>
<testsuites><testsuite name="pytest" errors="0" failures="0" skipped="1" tests="3" time="1.0">
<testcase classname="tests.ops.test_unary" name="test_hardswish_op[1048576-dtype0]" time="0.5">
<properties><property name="op" value="HardswishFwdOp"/><property name="max_abs_err" value="1.0e-03"/></properties>
</testcase>
<testcase classname="tests.ops.test_unary" name="test_hardswish_op[1048576-dtype1]" time="0.25">
<properties><property name="op" value="HardswishFwdOp"/><property name="max_abs_err" value="3.0e-03"/></properties>
</testcase>
<testcase classname="tests.ops.test_unary" name="test_skip" time="0"><skipped message="no gpu"/></testcase>
</testsuite></testsuites>
"""

JUNIT_FAIL = """<?xml version="1.0" encoding="utf-8"?>
<testsuite name="pytest" errors="1" failures="1" skipped="0" tests="2">
<testcase classname="tests.ops.test_unary" name="test_a"><failure message="mismatch">trace</failure></testcase>
</testsuite>
"""


def _record(op, case_id, label, ratio, mode="rocprof", tag="tileops", kernels=True):
    result = {"latency_us": 10.0, "Ratio(%)": ratio, "bandwidth_tbs": 6.0, "prof_mode": mode}
    if mode == "rocprof":
        result["rocprof"] = {"kernel_name_requested": None, "kernel_name_resolved": "tileops",
                             "kernels": [{"name": "tileops::k", "avg_us": 10.0}] if kernels else []}
    return {"operator": op, "case_id": case_id, "label": label, "params": {"shape": [4, 4]},
            "result": result, "tag": tag}


def test_parse_junit_preserves_properties(tmp_path):
    p = tmp_path / "c.xml"
    p.write_text(JUNIT_OK)
    r = parse_junit_report(p)
    assert r["status"] == "passed" and r["tests"] == 3 and r["passed"] == 2 and r["skipped"] == 1
    case = r["cases"][0]
    assert case["properties"] == {"op": "HardswishFwdOp", "max_abs_err": "1.0e-03"}
    assert case["nodeid"] == "tests.ops.test_unary::test_hardswish_op[1048576-dtype0]"
    assert r["cases"][2]["outcome"] == "skipped" and r["cases"][2]["message"] == "no gpu"


def test_parse_junit_counts_suite_level_errors(tmp_path):
    p = tmp_path / "c.xml"
    p.write_text(JUNIT_FAIL)
    r = parse_junit_report(p)
    assert r["status"] == "failed" and r["failed"] == 1 and r["errors"] == 1 and r["passed"] == 0
    assert parse_junit_report(tmp_path / "missing.xml")["status"] == "missing"


def test_benchmark_json_missing_and_present(tmp_path):
    assert load_benchmark_report(tmp_path / "b.json")["status"] == "missing"
    (tmp_path / "b.json").write_text(json.dumps({"schema_version": 1, "records": []}))
    assert load_benchmark_report(tmp_path / "b.json")["status"] == "present"


def test_analyzer_keeps_per_shape_ratio_and_filters():
    bench = {"status": "present", "profiling_mode_requested": "rocprof", "records": [
        _record("HardswishFwdOp", "a", "fc-wide", 80.0),
        _record("HardswishFwdOp", "b", "mbv3-stage2", 60.0),
        _record("HardswishFwdOp", "c", "smoke-1m", 10.0),          # smoke: dropped
        _record("HardswishFwdOp", "d", "fc-wide", 1.0, tag="torch"),  # not tileops: dropped
    ]}
    corr = {"status": "passed", "tests": 2, "passed": 2, "failed": 0, "errors": 0, "cases": []}
    run = analyzer.analyze_run(operator="HardswishFwdOp", correctness=corr, correctness_exit_code=0,
                               benchmark=bench, benchmark_exit_code=0,
                               benchmark_tests={"tests": 2, "failed": 0, "errors": 0, "cases": []})
    assert run["status"] == "passed"
    ratios = sorted(c["roofline_utilization_percent"] for c in run["performance"]["cases"])
    assert ratios == [60.0, 80.0]
    assert run["operators"][0]["ratio_range"] == {"min": 60.0, "max": 80.0}


def test_analyzer_flags_profiler_fallback_and_empty_capture():
    bench = {"status": "present", "profiling_mode_requested": "rocprof", "records": [
        _record("HardswishFwdOp", "a", "fc-wide", 80.0, mode="events"),
        _record("HardswishFwdOp", "b", "big", 70.0, kernels=False),
    ]}
    corr = {"status": "passed", "tests": 1, "passed": 1, "failed": 0, "errors": 0, "cases": []}
    run = analyzer.analyze_run(operator="HardswishFwdOp", correctness=corr, correctness_exit_code=0,
                               benchmark=bench, benchmark_exit_code=0)
    assert run["status"] == "partial"
    assert run["summary"]["profiler_fallback_count"] == 1
    assert run["summary"]["invalid_profile_count"] == 1
    assert any("requested rocprof but recorded events" in w for w in run["warnings"])


def test_analyzer_multi_operator_summary(tmp_path):
    p = tmp_path / "c.xml"
    p.write_text(JUNIT_OK)
    corr = parse_junit_report(p)
    catalog = runner.list_operators()
    bench = {"status": "present", "profiling_mode_requested": "rocprof", "records": [
        _record("HardswishFwdOp", "a", "fc-wide", 80.0), _record("IsnanFwdOp", "b", "16m", 70.0)]}
    run = analyzer.analyze_run(operator="all", correctness=corr, correctness_exit_code=0,
                               benchmark=bench, benchmark_exit_code=0, operator_catalog=catalog)
    by = {o["operator"]: o for o in run["operators"]}
    assert len(by) == len(catalog)
    assert by["HardswishFwdOp"]["cases"] == 2 and by["HardswishFwdOp"]["passed"] == 2
    assert by["HardswishFwdOp"]["avg_max_abs_err"] == pytest.approx(2e-3)
    assert by["IsnanFwdOp"]["performance_cases"] == 1 and by["IsnanFwdOp"]["cases"] == 0
    assert run["status"] == "passed"


def test_correctness_failure_fails_run():
    corr = {"status": "failed", "tests": 1, "passed": 0, "failed": 1, "errors": 0, "cases": []}
    run = analyzer.analyze_run(operator="X", correctness=corr, correctness_exit_code=1)
    assert run["status"] == "failed" and not run["summary"]["benchmark_requested"]


def test_write_reports_creates_all_formats(tmp_path):
    bench = {"status": "present", "profiling_mode_requested": "rocprof", "records": [
        _record("HardswishFwdOp", "a", "fc-<wide>|x", 80.0)]}
    corr = {"status": "failed", "tests": 1, "passed": 0, "failed": 1, "errors": 0,
            "cases": [{"nodeid": "t::a", "outcome": "failed", "message": "boom <b>"}]}
    run = analyzer.analyze_run(operator="HardswishFwdOp", correctness=corr, correctness_exit_code=1,
                               benchmark=bench, benchmark_exit_code=None)
    paths = write_reports(run, tmp_path / "out")
    assert json.loads(paths["json"].read_text())["schema_version"] == 2
    md = paths["markdown"].read_text()
    assert "# TileOPs Evaluation Report: HardswishFwdOp" in md and "fc-<wide>\\|x" in md
    assert "## Failed Cases" in md and "boom <b>" in md
    page = paths["html"].read_text()
    assert page.startswith("<!DOCTYPE html>") and "boom &lt;b&gt;" in page and "<script" not in page


def test_render_upgrades_legacy_run_json():
    legacy = {"operator": "IsnanFwdOp", "status": "passed",
              "correctness": {"tests": 4, "passed": 4, "failed": 0, "errors": 0, "cases": []},
              "performance": {"cases": [{"operator": "IsnanFwdOp", "label": "16m",
                                         "roofline_utilization_percent": 70.0, "params": {}}]}}
    md = render_markdown(legacy)
    assert "| IsnanFwdOp | 100.0% (4/4)" in md and "70.00%" in md
    assert "IsnanFwdOp" in render_html(legacy)


def _fake_stages(monkeypatch, correctness_xml, bench_records, calls):
    def fake(*, root, target, junit_path, log_path, env, pytest_args, timeout):
        calls.append({"target": target, "args": list(pytest_args), "env": dict(env)})
        log_path.write_text("fake\n")
        if "benchmarks" in target:
            junit_path.write_text(JUNIT_OK.replace('skipped="1"', 'skipped="0"'))
            report = Path(env["TILEOPS_BENCHMARK_REPORT_PATH"]).with_suffix(".json")
            report.write_text(json.dumps({"schema_version": 1, "profiling_mode_requested":
                                          env["TILEOPS_PROF_MODE"], "records": bench_records}))
            return 0, ["pytest", target]
        junit_path.write_text(correctness_xml)
        return (0 if correctness_xml == JUNIT_OK else 1), ["pytest", target]

    monkeypatch.setattr(runner, "_run_pytest", fake)


def test_runner_gates_benchmark_and_writes_report(tmp_path, monkeypatch):
    calls = []
    _fake_stages(monkeypatch, JUNIT_OK, [_record("HardswishFwdOp", "a", "fc-wide", 80.0)], calls)
    run, run_dir, code = runner.run_operator("HardswishFwdOp", reports_dir=tmp_path / "r",
                                             pytest_args=["-m", "full"])
    assert code == 0 and run["status"] == "passed"
    assert [c["target"] for c in calls] == ["tests/ops/test_unary.py",
                                            "tile-ascendnpu-ops_amd/benchmarks/ops/bench_hardswish.py"]
    assert calls[0]["args"][-2:] == ["-k", "hardswish or activation or unary"]
    assert calls[1]["args"] == ["-m", "(full) and not smoke"]
    assert calls[1]["env"]["TILEOPS_PROF_MODE"] == "rocprof"
    for f in ("run.json", "report.md", "report.html"):
        assert (run_dir / f).exists()
    latest = json.loads((tmp_path / "r" / "latest.json").read_text())
    assert latest["run_id"] == run_dir.name


def test_runner_skips_benchmark_after_correctness_failure(tmp_path, monkeypatch):
    calls = []
    _fake_stages(monkeypatch, JUNIT_FAIL, [], calls)
    run, _dir, code = runner.run_operator("IsnanFwdOp", reports_dir=tmp_path / "r")
    assert code == 1 and run["status"] == "failed" and len(calls) == 1
    assert run["benchmark_tests"]["status"] == "skipped"


def test_runner_merges_user_keyword(tmp_path, monkeypatch):
    calls = []
    _fake_stages(monkeypatch, JUNIT_OK, [_record("IsnanFwdOp", "a", "16m", 70.0)], calls)
    runner.run_operator("IsnanFwdOp", reports_dir=tmp_path / "r", pytest_args=["-k", "1048576"])
    assert calls[0]["args"] == ["-k", "(1048576) and (isnan or predicates or predicate_fp32)"]
    assert calls[1]["args"] == ["-k", "1048576", "-m", "not smoke"]


def test_all_mode_and_unknown_operator():
    assert runner.resolve_operator("all") == ("tests/ops", "tile-ascendnpu-ops_amd/benchmarks/ops")
    with pytest.raises(ValueError, match="source.test/source.bench"):
        runner.resolve_operator("NoSuchOp")
    assert runner.resolve_operator("NoSuchOp", test_file="a", benchmark_file="b") == ("a", "b")


@pytest.mark.parametrize("args, addopts", [(["-n", "4"], None), (["-n4"], None),
                                           (["--numprocesses=2"], None), ([], "-n 3")])
def test_runner_rejects_xdist(args, addopts):
    with pytest.raises(ValueError, match="xdist"):
        runner._reject_xdist(args, addopts)


def test_runner_allows_serial_xdist_flags():
    runner._reject_xdist(["-n", "0", "-n0", "--numprocesses=0"], None)


def test_exclude_smoke_needs_expression():
    with pytest.raises(ValueError, match="requires a marker expression"):
        runner._exclude_smoke(["-m"])
    assert runner._exclude_smoke(["--markexpr=a", "-x"]) == ["-x", "-m", "(a) and not smoke"]


def test_cli_list_and_render(tmp_path, capsys):
    assert cli.main(["list"]) == 0
    out = capsys.readouterr().out
    assert "GatedDeltaNetPrefillFwdOp" in out and "family=attention" in out
    corr = {"status": "passed", "tests": 1, "passed": 1, "failed": 0, "errors": 0, "cases": []}
    run = analyzer.analyze_run(operator="IsnanFwdOp", correctness=corr, correctness_exit_code=0)
    (tmp_path / "run.json").write_text(json.dumps(run))
    assert cli.main(["render", str(tmp_path / "run.json"), "--output-dir", str(tmp_path / "o")]) == 0
    assert (tmp_path / "o" / "report.html").exists()
    with pytest.raises(SystemExit):
        cli.main(["run", "--op", "X", "--prof-mode", "msprof"])


def test_benchmark_report_writes_markdown_and_json(tmp_path, monkeypatch):
    bb.BenchmarkReport.clear()
    monkeypatch.setenv("PYTEST_CURRENT_TEST", "bench_x.py::test_b[fc-wide-float16] (call)")
    bb.BenchmarkReport.record("HardswishFwdOp", {"shape": (2048, 4096), "dtype": torch.float16,
                                                 "op": object(), "_private": 1},
                              {"latency_us": 12.5, "Ratio(%)": 70.0, "prof_mode": "events"})
    bb.BenchmarkReport.set_prof_mode("events")
    bb.BenchmarkReport.dump(str(tmp_path / "bench.md"))
    data = json.loads((tmp_path / "bench.json").read_text())
    (rec,) = data["records"]
    assert rec["operator"] == "HardswishFwdOp" and rec["label"] == "fc-wide"
    assert rec["params"] == {"dtype": "float16", "shape": [2048, 4096]}
    assert rec["case_id"].startswith("HardswishFwdOp-") and len(rec["case_id"]) == len("HardswishFwdOp-") + 12
    assert data["profiling_mode_requested"] == "events"
    md = (tmp_path / "bench.md").read_text()
    assert "## HardswishFwdOp" in md and "| fc-wide | 12.5000 | 70.0000 |" in md
    bb.BenchmarkReport.clear()


def test_roofline_metrics_closed_form():
    # 8 GB moved in 1.25 ms at 8 TB/s peak -> 80% of the HBM roofline
    m = bb.roofline_metrics(flops=1e9, nbytes=8e9, latency_ms=1.25, dtype=torch.bfloat16)
    assert m["Bandwidth(TB/s)"] == pytest.approx(6.4)
    assert m["Ratio(%)"] == pytest.approx(80.0) and m["bound"] == "memory"
    # 2.5166 PFLOP in 2 s at the bf16 MFMA peak -> 50%
    m = bb.roofline_metrics(flops=2516.6e12, nbytes=1e9, latency_ms=2000.0, dtype=torch.bfloat16)
    assert m["Ratio(%)"] == pytest.approx(50.0) and m["bound"] == "compute"
    assert bb.compute_peak_tflops(torch.float32) == 157.3


def test_profile_log_path_is_session_stable(monkeypatch):
    bb.BenchmarkReport.clear()
    a = bb.profile_run_log_path("rocprof")
    assert a.startswith("profile_run_rocprof_") and a.endswith(".log")
    assert bb.profile_run_log_path("rocprof") == a
    assert bb.profile_run_json_path("rocprof") == a[:-4] + ".json"
    bb.BenchmarkReport.clear()


def test_rocprof_per_call_split():
    d = [("tileops::prep", 0, 1000), ("tileops::main", 1000, 4000)] * 4
    calls, per = rp.per_call_latency_us(d, n_calls=3, n_total_calls=4)
    assert per == 2 and calls == [4.0, 4.0, 4.0]
    with pytest.raises(ValueError, match="do not split"):
        rp.per_call_latency_us(d[:-1], n_calls=3, n_total_calls=4)


def test_rocprof_script_rebuilds_op():
    from tileops.ops.elementwise.clamp_scalar import ClampScalarFwdOp

    op = ClampScalarFwdOp(N_total=4096, dtype=torch.bfloat16, min=-1.0, max=None)
    args = rp._extract_op_init_args(op)
    assert args == {"N_total": 4096, "dtype": torch.bfloat16, "min": -1.0, "max": None}
    src = rp._generate_script(op, "/x/inputs.pt", 5, 10, 0)
    ctor = [line for line in src.splitlines() if line.startswith("fn = ")][0][5:]
    again = eval(ctor, {"ClampScalarFwdOp": ClampScalarFwdOp, "torch": torch})  # noqa: S307
    assert rp._extract_op_init_args(again) == args
    assert "weights_only=True" in src and "range(5)" in src and "range(10)" in src


def test_counter_runs_use_fixed_call_counts(monkeypatch):
    # the counter passes divide their totals by warm_up + launch_count, so
    # their child program must not settle; exercised with the rocprofv3
    # runs replaced by stand-ins
    from tileops.ops.elementwise.clamp_scalar import ClampScalarFwdOp

    scripts = []

    def fake_run(script, counters, work, timeout, env):
        scripts.append(open(script).read())
        return "db"

    totals = {"FETCH_SIZE": 4.0 * 8, "WRITE_SIZE": 2.0 * 8, "SQ_VALU_MFMA_BUSY_CYCLES": 0.0,
              "GRBM_GUI_ACTIVE": 8.0}
    monkeypatch.setattr(rp, "counter_calibration", lambda timeout=300: (2.0, 1.0))
    monkeypatch.setattr(rp, "_run_pmc", fake_run)
    monkeypatch.setattr(rp, "read_counter_totals", lambda db, regex: dict(totals))
    op = ClampScalarFwdOp(N_total=4096, dtype=torch.bfloat16, min=-1.0, max=None)
    res = rp.bench_kernel_counters(op, (torch.zeros(4096, dtype=torch.bfloat16),),
                                   launch_count=3, warm_up=1)
    assert len(scripts) == len(rp.COUNTER_PASSES)
    assert all("< 0.0:" in src for src in scripts)  # no settle time
    assert res["hbm_read_bytes"] == 4 * 8 * 1024 * 2 // 4
    assert res["hbm_write_bytes"] == 2 * 8 * 1024 // 4


def test_rocprof_script_settles_and_counts_its_calls(capsys):
    # the child runs warm-up, then untimed batches for the settle time, then
    # the measured calls, and prints the total that the parent splits the
    # dispatches by; run here against a stand-in for torch
    import types

    class Fn:
        def __init__(self):
            self.n = 0

        def __call__(self, *a):
            self.n += 1

    fake_cuda = types.SimpleNamespace(set_device=lambda i: None, synchronize=lambda: None)
    fake_torch = types.SimpleNamespace(cuda=fake_cuda, Tensor=torch.Tensor, no_grad=torch.no_grad,
                                       load=lambda path, weights_only: [1.0])
    src = rp._generate_script(Fn, "/x/inputs.pt", 3, 7, 0, settle_s=0.05)
    body = "\n".join(line for line in src.splitlines()
                     if not line.startswith(("import torch", "from ", "fn = ")))
    fn = Fn()
    exec(body, {"torch": fake_torch, "fn": fn})  # noqa: S102
    out = capsys.readouterr().out
    total = int(out.split("tileops-rocprof: calls ")[1].split()[0])
    assert total == fn.n and total >= 3 + 3 + 7  # at least one settle batch of warm_up calls
    assert (total - 7 - 3) % 3 == 0
    assert "tileops-rocprof: done" in out


def test_rocprof_rejects_closures():
    with pytest.raises(TypeError, match="events mode"):
        rp.bench_kernel_rocprof(lambda x: x, (torch.zeros(1),))


def test_analyzer_attributes_cases_of_shared_test_files():
    """Cases of a test file that several ops share go to the op whose class
    name is in the case id, else the one whose test_keyword matches."""
    catalog = [
        {"name": "AddFwdOp", "test": "tests/ops/test_add_sub.py"},
        {"name": "SubFwdOp", "test": "tests/ops/test_add_sub.py"},
        {"name": "LerpFwdOp", "test": "tests/ops/test_lerp.py", "test_keyword": "lerp_scalar"},
        {"name": "LerpTensorFwdOp", "test": "tests/ops/test_lerp.py", "test_keyword": "lerp_tensor"},
    ]
    case = lambda cls, name: {"classname": cls, "name": name}  # noqa: E731
    pick = lambda c: analyzer._case_operator(c, catalog, None)  # noqa: E731
    assert pick(case("tests.ops.test_add_sub", "test_add_sub[1-dtype0-shapes0-SubFwdOp--1.0]")) == "SubFwdOp"
    assert pick(case("tests.ops.test_add_sub", "test_add_sub[1-dtype0-shapes0-AddFwdOp-1.0]")) == "AddFwdOp"
    assert pick(case("tests.ops.test_lerp", "test_lerp_scalar_weights[0.3-dtype1]")) == "LerpFwdOp"
    assert pick(case("tests.ops.test_lerp", "test_lerp_tensor[shapes0-dtype0]")) == "LerpTensorFwdOp"
    assert pick(case("tests.ops.test_lerp", "test_lerp_dtype_mismatch_rejected")) is None


def test_setup_gpu_label_from_gpu_agents(monkeypatch):
    """The GPU label comes from rocminfo's GPU agent, not the CPU agent."""
    from tileops.reporting import setup_info

    out = ("*******\nAgent 1\n*******\n  Name:                    AMD EPYC 9575F\n"
           "  Marketing Name:          AMD EPYC 9575F\n  Device Type:             CPU\n"
           "*******\nAgent 2\n*******\n  Name:                    gfx950\n"
           "  Marketing Name:          AMD Instinct MI355X\n  Device Type:             GPU\n")

    class _Res:
        stdout = out

    monkeypatch.setattr(setup_info.subprocess, "run", lambda *a, **k: _Res())
    assert setup_info._gpu_info() == "AMD Instinct MI355X (gfx950) x 1"


def test_runner_with_counters_sets_the_benchmark_env(tmp_path, monkeypatch):
    calls = []
    rec = _record("HardswishFwdOp", "a", "fc-wide", 80.0)
    rec["result"].update({"HBM bytes (counters)": 60_000_000, "HBM(TB/s, counters)": 6.0,
                          "MFMA busy(%)": 0.0})
    _fake_stages(monkeypatch, JUNIT_OK, [rec], calls)
    run, run_dir, code = runner.run_operator("HardswishFwdOp", reports_dir=tmp_path / "r",
                                             with_counters=True)
    assert code == 0
    assert calls[1]["env"]["TILEOPS_ROCPROF_COUNTERS"] == "1"
    case = run["performance"]["cases"][0]
    assert case["hbm_bytes_measured"] == 60_000_000 and case["mfma_busy_percent"] == 0.0
    md = (run_dir / "report.md").read_text()
    assert "HBM (TB/s, counters)" in md and "MFMA busy (%)" in md
    # bandwidth 6 TB/s x 10 us = 60,000,000 roofline bytes: ratio 1.000
    assert "1.000" in md
    calls.clear()
    runner.run_operator("HardswishFwdOp", reports_dir=tmp_path / "r2")
    assert "TILEOPS_ROCPROF_COUNTERS" not in calls[1]["env"]


def test_counter_totals_from_a_pmc_database(tmp_path):
    import sqlite3

    db = tmp_path / "pmc_results.db"
    con = sqlite3.connect(db)
    con.execute("create table counters_collection (kernel_name text, counter_name text, value real)")
    con.executemany("insert into counters_collection values (?, ?, ?)", [
        ("void tileops::gdn::gdn_fused_kernel<8>(tileops::gdn::Args)", "FETCH_SIZE", 100.0),
        ("void tileops::gdn::gdn_fused_kernel<4>(tileops::gdn::Args)", "FETCH_SIZE", 50.0),
        ("void tileops::gdn::gdn_fused_kernel<8>(tileops::gdn::Args)", "FETCH_SIZE", 100.0),
        ("void at::native::copy_kernel", "FETCH_SIZE", 999.0),
        ("void tileops::gdn::gdn_fused_kernel<4>(tileops::gdn::Args)", "GRBM_GUI_ACTIVE", 8000.0),
    ])
    con.commit()
    con.close()
    tot = rp.read_counter_totals(str(db), "tileops")
    assert tot == {"FETCH_SIZE": 250.0, "GRBM_GUI_ACTIVE": 8000.0}
    assert rp.read_counter_totals(str(db), "gdn_fused_kernel<4>") == {"FETCH_SIZE": 50.0,
                                                                     "GRBM_GUI_ACTIVE": 8000.0}


def test_profile_attaches_counters_when_asked(monkeypatch):
    """rocprof mode with TILEOPS_ROCPROF_COUNTERS=1: the counter summary lands in
    the result next to the latency (measured bytes over the latency)."""
    meta = {"kernel_name_resolved": "tileops", "kernels": []}
    monkeypatch.setattr(rp, "bench_kernel_rocprof", lambda f, args=(): (0.01, "/tmp", dict(meta)))
    monkeypatch.setattr(rp, "bench_kernel_counters",
                        lambda f, args=(), kernel_name=None: {"hbm_bytes": 80_000_000,
                                                              "mfma_busy_percent": 12.5})
    monkeypatch.setattr(bb, "get_device_backend", lambda: type("B", (), {"synchronize": lambda s: None})())
    monkeypatch.setenv("TILEOPS_ROCPROF_COUNTERS", "1")

    class _Bench(bb.BenchmarkBase):
        def calculate_flops(self):
            return None

        def calculate_memory(self):
            return 80_000_000

    res = _Bench(type("W", (), {"dtype": torch.float16})()).profile(lambda: None, mode="rocprof")
    assert res["prof_mode"] == "rocprof"
    assert res["HBM bytes (counters)"] == 80_000_000
    assert res["HBM(TB/s, counters)"] == pytest.approx(8.0)  # 80 MB in 10 us
    assert res["MFMA busy(%)"] == 12.5


def test_profile_records_why_rocprof_or_counters_failed(monkeypatch):
    """A rocprof failure falls back to events timing with its reason in the
    result; a counter failure keeps the rocprof timing and records the error;
    the analyzer turns both into warnings."""
    monkeypatch.setattr(bb, "get_device_backend", lambda: type("B", (), {"synchronize": lambda s: None})())
    monkeypatch.setattr(bb, "bench_kernel", lambda f, args=(): 0.02)

    class _Bench(bb.BenchmarkBase):
        def calculate_flops(self):
            return None

        def calculate_memory(self):
            return 1_000_000

    bench = _Bench(type("W", (), {"dtype": torch.float16})())

    def _fail(f, args=()):
        raise ValueError("0 matching dispatches do not split into 15 calls")

    monkeypatch.setattr(rp, "bench_kernel_rocprof", _fail)
    res = bench.profile(lambda: None, mode="rocprof")
    assert res["prof_mode"] == "events" and "rocprof" not in res
    assert "0 matching dispatches" in res["rocprof_fallback"]

    meta = {"kernels": [{"name": "tileops::k", "avg_us": 10.0}]}
    monkeypatch.setattr(rp, "bench_kernel_rocprof", lambda f, args=(): (0.01, "/tmp", dict(meta)))

    def _ctr_fail(f, args=(), kernel_name=None):
        raise RuntimeError("rocprofv3 --pmc failed (exit 1)")

    monkeypatch.setattr(rp, "bench_kernel_counters", _ctr_fail)
    monkeypatch.setenv("TILEOPS_ROCPROF_COUNTERS", "1")
    res2 = bench.profile(lambda: None, mode="rocprof")
    assert res2["prof_mode"] == "rocprof" and res2["latency_us"] == pytest.approx(10.0)
    assert "--pmc failed" in res2["rocprof"]["counters_error"]
    assert "HBM bytes (counters)" not in res2

    bench = {"status": "present", "profiling_mode_requested": "rocprof", "records": [
        {"operator": "Op", "case_id": "a", "label": "big", "result": res, "tag": "tileops"},
        {"operator": "Op", "case_id": "b", "label": "big", "result": res2, "tag": "tileops"}]}
    corr = {"status": "passed", "tests": 1, "passed": 1, "failed": 0, "errors": 0, "cases": []}
    run = analyzer.analyze_run(operator="Op", correctness=corr, correctness_exit_code=0,
                               benchmark=bench, benchmark_exit_code=0)
    text = " ".join(run["warnings"])
    assert "requested rocprof but recorded events (ValueError: 0 matching" in text
    assert "counter collection failed (RuntimeError: rocprofv3 --pmc failed" in text


def test_declared_kernel_regexes_match_mangled_and_demangled_names():
    """rocprofv3 stores the demangled name where its demangler succeeds and the
    mangled one where it does not; every declared regex matches both."""
    import re

    from tileops.kernels.attention.multi_head_attention.multi_head_attention import (
        GQAPrefillFwdKernel,
    )
    from tileops.kernels.linear_attention.gdn_prefill.gdn_prefill import GDNPrefillFwdKernel

    gdn = re.compile(GDNPrefillFwdKernel.profile_kernel_name)
    assert gdn.search("void tileops::gdn::gdn_fused_kernel<4>(tileops::gdn::Args)")
    assert gdn.search("_ZN7tileops3gdn16gdn_fused_kernelILi8EEEvNS0_4ArgsE")
    assert gdn.search("_ZN7tileops3gdn21gdn_copy_state_kernelEPKfPfl")
    mha = re.compile(GQAPrefillFwdKernel.profile_kernel_name)
    assert mha.search("_ZN7tileops3mha14mha_fwd_kernelIDF16_Li64ELi64ELb1ELi64ELb0EEEvPKT_")
    assert mha.search("void tileops::mha::mha_fwd_kernel<float, 64>(float const*)")
    assert not mha.search("void at::native::elementwise_kernel<128, 4>()")
