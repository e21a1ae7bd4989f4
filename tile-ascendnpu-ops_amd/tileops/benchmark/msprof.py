"""Names of the reference's ``tileops.benchmark.msprof`` module, on rocprofv3.

Callers written against the reference import these by module path
(examples/TileOPs/tileops/benchmark/msprof.py:51,108,251,419; the test files
tests/ops/test_gelu_and_mul.py:23 and tests/reporting/test_reporting.py:5):

* ``_extract_op_init_args`` -- the constructor arguments an Op can be rebuilt
  from in a profiler subprocess (the rocprof path's own function);
* ``bench_kernel_msprof`` -- kernel-only latency of an Op or module-level
  callable.  On this GPU it runs ``rocprofv3 --kernel-trace`` through
  :func:`tileops.benchmark.rocprof.bench_kernel_rocprof` and returns
  ``(latency_ms, output_dir)`` as the msprof version did;
* ``_parse_op_basic_info`` -- reads the ``OpBasicInfo*.csv`` files an
  ``msprof op`` run leaves (one ``Task Duration(us)`` row per captured
  dispatch), so profiles recorded on the reference's hardware can still be
  loaded next to rocprof results.
"""

from __future__ import annotations

import csv
import logging
from pathlib import Path
from typing import Callable, Optional

from tileops.benchmark.rocprof import _extract_op_init_args, bench_kernel_rocprof

__all__ = ["bench_kernel_msprof", "_extract_op_init_args", "_parse_op_basic_info"]

_logger = logging.getLogger("tileops.benchmark.msprof")

_DURATION = "Task Duration(us)"
_NAME = "Op Name"


def _parse_op_basic_info(output_dir: str) -> tuple[list[float], str, list[str]]:
    """``(durations_us, first_op_name, sorted_distinct_op_names)`` from every
    ``OpBasicInfo*.csv`` below ``output_dir``.

    Files are read in sorted path order (an msprof run writes
    ``OPPROF_*/<op>/<index>/OpBasicInfo_<ts>.csv``), so durations and the
    first name follow that order.  Raises ``FileNotFoundError`` when there is
    no such file and ``ValueError`` when none holds a duration; a
    non-numeric duration is logged and skipped."""
    root = Path(output_dir)
    files = sorted(str(p) for p in root.rglob("OpBasicInfo*.csv") if p.is_file())
    if not files:
        raise FileNotFoundError(f"No OpBasicInfo*.csv found under {output_dir}")
    durations: list[float] = []
    first = ""
    seen: set[str] = set()
    for path in files:
        with open(path, newline="", encoding="utf-8") as fh:
            for row in csv.DictReader(fh):
                raw = (row.get(_DURATION) or "").strip()
                if raw:
                    try:
                        durations.append(float(raw))
                    except ValueError:
                        _logger.warning("Non-numeric %s in %s: %r", _DURATION, path, raw)
                name = (row.get(_NAME) or "").strip()
                if name:
                    seen.add(name)
                    first = first or name
    if not durations:
        raise ValueError(f"No {_DURATION} values found in OpBasicInfo CSVs under {output_dir}")
    return durations, first, sorted(seen)


def bench_kernel_msprof(
    functor: Callable,
    args: tuple = (),
    *,
    kernel_name: Optional[str] = None,
    launch_count: Optional[int] = None,
    warm_up: Optional[int] = None,
    output_dir: Optional[str] = None,
    keep_output: bool = False,
) -> tuple[float, str]:
    """Kernel-only latency (ms) of ``functor(*args)`` and the profile
    directory, measured by rocprofv3.  ``keep_output`` keeps the result
    database (it is removed otherwise unless ``output_dir`` is given)."""
    if keep_output and output_dir is None:
        import tempfile

        output_dir = tempfile.mkdtemp(prefix="tileops_rocprof_keep_")
    latency_ms, out, _meta = bench_kernel_rocprof(
        functor, args, kernel_name=kernel_name, launch_count=launch_count, warm_up=warm_up,
        output_dir=output_dir)
    return latency_ms, out
