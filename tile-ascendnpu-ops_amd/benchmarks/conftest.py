"""Benchmark-suite session hooks (layout of examples/TileOPs/benchmarks/conftest.py).

Seeds every case with the reference's seed, clears the report at session
start and dumps it (Markdown + JSON) at session end, copies each case's
headline figures into its JUnit properties, and collects ``bench_*.py``
files.  Benchmarks launch HIP kernels: they need a GPU.
"""

import gc
import os
import sys

import pytest
import torch

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if _PKG not in sys.path:
    sys.path.insert(0, _PKG)

from tileops.benchmark.benchmark_base import BenchmarkReport, _bench_results  # noqa: E402
from tileops.device import get_device_backend  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (launches HIP kernels)")


def pytest_collection_modifyitems(config, items):
    # every benchmark case launches HIP kernels: `-m "not gpu"` deselects them
    here = os.path.dirname(os.path.abspath(__file__))
    for item in items:
        if str(item.fspath).startswith(here):
            item.add_marker(pytest.mark.gpu)


def pytest_collect_file(file_path, parent):
    # files named on the command line are collected by pytest itself
    if (file_path.suffix == ".py" and file_path.name.startswith("bench_")
            and not parent.session.isinitpath(file_path)):
        return pytest.Module.from_parent(parent, path=file_path)
    return None


@pytest.fixture(autouse=True)
def setup() -> None:
    torch.manual_seed(1235)
    get_device_backend().manual_seed_all(1235)


def pytest_sessionstart(session):
    BenchmarkReport.clear()


def pytest_sessionfinish(session, exitstatus):
    BenchmarkReport.set_prof_mode(os.environ.get("TILEOPS_PROF_MODE", "rocprof"))
    BenchmarkReport.dump()


@pytest.hookimpl(hookwrapper=True)
def pytest_runtest_call(item):
    _bench_results.entries = []
    try:
        yield
        entry = next((e for e in getattr(_bench_results, "entries", [])
                      if e["tag"].startswith("tileops")), None)
        if entry:
            item.user_properties.append(("op", entry["op"]))
            if "op_module" in entry:
                item.user_properties.append(("op_module", entry["op_module"]))
            item.user_properties.append(("tileops_latency_us", f"{entry.get('latency_us', 0):.4f}"))
            for key, prop in (("tflops", "tileops_tflops"), ("bandwidth_tbs", "tileops_bandwidth_tbs"),
                              ("Ratio(%)", "tileops_roofline_percent")):
                if entry.get(key) is not None:
                    item.user_properties.append((prop, f"{entry[key]:.2f}"))
    finally:
        _bench_results.entries = []
        gc.collect()
        backend = get_device_backend()
        if backend.is_available():
            backend.empty_cache()
