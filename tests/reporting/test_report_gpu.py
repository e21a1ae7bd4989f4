"""End-to-end report run on the GPU: correctness stage, then the benchmark
stage timed by rocprofv3 in child processes, then the run document."""

import pytest

from tileops.reporting import runner


@pytest.mark.gpu
def test_report_run_hardswish_rocprof(tmp_path):
    run, run_dir, code = runner.run_operator(
        "HardswishFwdOp", prof_mode="rocprof", reports_dir=tmp_path / "reports",
        pytest_args=["-k", "1048576 or fc-wide"], timeout=300)
    log = (run_dir / "pytest" / "benchmark.log")
    assert run["summary"]["correctness_passed"], (run_dir / "pytest" / "correctness.log").read_text()[-3000:]
    assert code == 0 and run["status"] == "passed", log.read_text()[-3000:] if log.exists() else run
    cases = run["performance"]["cases"]
    assert {c["label"] for c in cases} == {"fc-wide"} and len(cases) == 2
    for c in cases:
        assert c["prof_mode"] == "rocprof" and c["profiler_valid"]
        assert c["latency_us"] > 0 and 0 < c["roofline_utilization_percent"] < 100
        assert all("tileops" in k for k in c["kernels"])
    assert (run_dir / "report.html").exists()
