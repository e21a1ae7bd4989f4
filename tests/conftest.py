"""Shared pytest setup: import paths, markers, and the reference's seed.

The ``gpu`` marker tags tests that launch HIP kernels; everything else runs
on a host without a GPU (oracle pins, API contracts, C-ABI symbol checks).
"""

import os
import sys

import pytest
import torch

_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(_ROOT, "tile-ascendnpu-ops_amd"), _ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

from tileops.device import get_device_backend  # noqa: E402
from tileops.testing.test_base import get_check_result  # noqa: E402


def pytest_configure(config):
    for name, doc in (
        ("gpu", "needs an AMD GPU (launches HIP kernels)"),
        ("smoke", "fast critical-path tests"),
        ("full", "standard correctness coverage"),
        ("nightly", "exhaustive or long-running coverage"),
        ("packaging", "minimal install sanity check"),
    ):
        config.addinivalue_line("markers", f"{name}: {doc}")


@pytest.fixture(autouse=True)
def _seed() -> None:
    # seed of the reference suite (examples/TileOPs/tests/conftest.py:8-12)
    torch.manual_seed(1235)
    get_device_backend().manual_seed_all(1235)


@pytest.hookimpl(hookwrapper=True)
def pytest_runtest_call(item):
    yield
    cr = get_check_result()
    if cr.op_name:
        item.user_properties.append(("op", cr.op_name))
        if cr.op_module:
            item.user_properties.append(("op_module", cr.op_module))
        if cr.max_abs_err is not None:
            item.user_properties.append(("max_abs_err", f"{cr.max_abs_err:.2e}"))
        cr.op_name = None
        cr.op_module = None
        cr.max_abs_err = None
