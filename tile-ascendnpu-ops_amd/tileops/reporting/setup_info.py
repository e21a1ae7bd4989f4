"""Report metadata and the runtime environment (GPU, ROCm, torch, host).

Sections of the reference's setup block
(examples/TileOPs/tileops/reporting/setup_info.py:136-171), with the NPU
fields replaced by their ROCm counterparts.  Nothing here initialises the
GPU: the device is read from ``rocminfo`` text, not through HIP.
"""

from __future__ import annotations

import importlib.metadata
import os
import platform
import re
import subprocess
import sys
from datetime import datetime
from pathlib import Path
from typing import Any


def _package_version(name: str) -> str | None:
    try:
        return importlib.metadata.version(name)
    except importlib.metadata.PackageNotFoundError:
        return None


def _rocm_version() -> str | None:
    for p in (Path("/opt/rocm/.info/version"), Path("/opt/rocm/.info/version-dev")):
        try:
            text = p.read_text(encoding="utf-8").strip()
        except OSError:
            continue
        if text:
            return text
    return os.environ.get("ROCM_VERSION")


def _gpu_info() -> str | None:
    try:
        out = subprocess.run(["rocminfo"], capture_output=True, text=True, timeout=20,
                             check=False).stdout
    except (OSError, subprocess.SubprocessError):
        return None
    # one block per agent; the GPU agents carry "Device Type: GPU"
    gpus = []
    for block in re.split(r"\n\*+\s*\n\s*Agent \d+", out):
        if not re.search(r"Device Type:\s*GPU", block):
            continue
        arch = re.search(r"Name:\s*(gfx\w+)", block)
        name = re.search(r"Marketing Name:\s*(.+)", block)
        if arch:
            gpus.append(((name.group(1).strip() if name else "") or "AMD GPU", arch.group(1)))
    if not gpus:
        return None
    return f"{gpus[0][0]} ({gpus[0][1]}) x {len(gpus)}"


def _cpu_info() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text(encoding="utf-8").splitlines():
            if line.startswith("model name"):
                return f"{line.split(':', 1)[1].strip()} ({os.cpu_count()} threads)"
    except OSError:
        pass
    return platform.machine() or "unknown"


def _container_info() -> str | None:
    if os.environ.get("TILEOPS_IMAGE"):
        return os.environ["TILEOPS_IMAGE"]
    if Path("/.dockerenv").exists():
        return "container"
    try:
        cgroup = Path("/proc/1/cgroup").read_text(encoding="utf-8", errors="ignore")
    except OSError:
        return None
    return "container" if any(k in cgroup for k in ("docker", "containerd", "kubepods")) else None


def collect_setup_info(
    *,
    scope: str,
    run_id: str,
    generated_at: str,
    profiler: str,
    git_commit: str | None,
    test_target: str,
    benchmark_target: str,
) -> dict[str, dict[str, Any]]:
    """``{"metadata": {...}, "environment": {...}}`` for the report header."""
    return {
        "metadata": {
            "framework": "TileOPs (MI355X / HIP) reporting",
            "date": generated_at or datetime.now().astimezone().isoformat(),
            "evaluation_scope": scope,
            "benchmark": "TileOPs pytest operator suite",
            "profiler": profiler,
            "run_id": run_id,
            "git_commit": git_commit,
            "correctness_target": test_target,
            "benchmark_target": benchmark_target,
        },
        "environment": {
            "gpu": _gpu_info(),
            "cpu": _cpu_info(),
            "rocm": _rocm_version(),
            "pytorch": _package_version("torch"),
            "python": sys.version.split()[0],
            "os": platform.platform(),
            "container": _container_info(),
        },
    }


__all__ = ["collect_setup_info"]
