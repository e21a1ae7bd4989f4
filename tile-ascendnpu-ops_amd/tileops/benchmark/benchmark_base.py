"""Benchmark core: kernel timing, roofline metrics and the benchmark report.

Interface of the reference's module (examples/TileOPs/tileops/benchmark/benchmark_base.py):
``bench_kernel`` (:116-203), ``_bench_with_mode`` (:206-250),
``BenchmarkBase.profile`` / ``_build_result`` (:269-357),
``workloads_to_params`` (:505-534), ``ManifestBenchmark`` (:537-563),
``BenchmarkReport`` (:587-856) and the session-stable
``profile_run_{mode}_{stamp}.log`` / ``.json`` paths.

MI355X specifics:

- timing modes are ``rocprof`` (default: kernel-only device time measured by
  ``rocprofv3`` in a child process, :mod:`tileops.benchmark.rocprof`) and
  ``events`` (HIP events around each call on the current stream, with the
  256 MB Infinity Cache flushed before every iteration);
- every result carries roofline figures against MI355X's published peaks:
  HBM 8.0 TB/s; dense MFMA 2516.6 TFLOP/s for fp16 / bf16; fp32 vector
  157.3 TFLOP/s.  ``Ratio(%)`` is the roofline floor time (the larger of
  bytes / HBM peak and flops / compute peak) over the measured latency.
"""

from __future__ import annotations

import hashlib
import json
import logging
import os
import threading
from abc import ABC, abstractmethod
from datetime import datetime
from pathlib import Path
from typing import Any, Callable, Generic, Optional, TypeVar

import pytest
import torch

from tileops.device import get_device_backend
from tileops.manifest import (
    WORKLOAD_RESERVED_KEYS,
    load_manifest,
    load_workloads,
    single_input_workload_contract,
)

__all__ = [
    "HBM_PEAK_TBS",
    "BenchmarkBase",
    "BenchmarkReport",
    "ManifestBenchmark",
    "bench_kernel",
    "compute_peak_tflops",
    "profile_run_json_path",
    "profile_run_log_path",
    "roofline_metrics",
    "workloads_to_params",
]

W = TypeVar("W")
_logger = logging.getLogger("tileops.benchmark")
_bench_results = threading.local()

HBM_PEAK_TBS = 8.0
_COMPUTE_PEAK_TFLOPS = {
    torch.float16: 2516.6,
    torch.bfloat16: 2516.6,
    torch.float32: 157.3,
}
DEFAULT_PROF_MODE = "rocprof"

_stamp: Optional[str] = None
_stamp_lock = threading.Lock()


def _prof_mode(mode: Optional[str] = None) -> str:
    return (mode or os.environ.get("TILEOPS_PROF_MODE", DEFAULT_PROF_MODE)).lower().strip()


def profile_run_log_path(prof_mode: Optional[str] = None) -> str:
    """``profile_run_{mode}_{YYYYmmdd_HHMMSS}.log``; the stamp is fixed at
    first use in the process (reset by ``BenchmarkReport.clear``)."""
    global _stamp
    with _stamp_lock:
        if _stamp is None:
            _stamp = datetime.now().strftime("%Y%m%d_%H%M%S")
        stamp = _stamp
    return f"profile_run_{_prof_mode(prof_mode)}_{stamp}.log"


def profile_run_json_path(prof_mode: Optional[str] = None) -> str:
    """The JSON companion of :func:`profile_run_log_path`."""
    return str(Path(profile_run_log_path(prof_mode)).with_suffix(".json"))


def compute_peak_tflops(dtype: Optional[torch.dtype]) -> float:
    """Dense compute peak for work carried out in ``dtype`` (fp32 if unknown)."""
    return _COMPUTE_PEAK_TFLOPS.get(dtype, _COMPUTE_PEAK_TFLOPS[torch.float32])


def roofline_metrics(flops: Optional[float], nbytes: Optional[float], latency_ms: float,
                     dtype: Optional[torch.dtype]) -> dict[str, Any]:
    """Roofline figures of one measured call (see the module docstring)."""
    out: dict[str, Any] = {}
    if latency_ms <= 0:
        return out
    seconds = latency_ms * 1e-3
    peak_tf = compute_peak_tflops(dtype)
    t_mem = (nbytes or 0) / (HBM_PEAK_TBS * 1e12)
    t_cmp = (flops or 0) / (peak_tf * 1e12)
    if nbytes:
        out["Bandwidth(TB/s)"] = nbytes / seconds * 1e-12
    if flops:
        out["Perf(TOps/s)"] = flops / seconds * 1e-12
    if flops and nbytes:
        out["AI(Ops/Byte)"] = flops / nbytes
    out["Computility(TOPs/s)"] = peak_tf
    out["Peak bandwidth(TB/s)"] = HBM_PEAK_TBS
    if t_mem or t_cmp:
        out["Ratio(%)"] = max(t_mem, t_cmp) / seconds * 100.0
        out["bound"] = "memory" if t_mem >= t_cmp else "compute"
    return out


def _workload_contract(op_name: str) -> tuple[str, frozenset[str]]:
    sig = load_manifest()[op_name].get("signature") or {}
    contract = single_input_workload_contract(sig)
    if contract is None:
        raise KeyError(
            f"workloads_to_params({op_name!r}) needs exactly one manifest "
            "tensor input; multi-input ops use their own bench files."
        )
    return contract


def bench_kernel(
    fn: Callable,
    args: tuple[Any, ...] = (),
    n_warmup: int = 5,
    n_repeat: int = 10,
    n_trials: int = 3,
) -> float:
    """Latency of ``fn(*args)`` in milliseconds from device events.

    ``n_warmup`` untimed calls, then ``n_trials`` trials of ``n_repeat``
    calls, each bracketed by events on the current stream after a cache
    flush and a synchronisation; inputs rotate over three clones (when
    they total at most 1 GiB) so consecutive calls see fresh addresses.
    Returns the median of the trial means."""
    if not isinstance(args, tuple):
        raise TypeError(f"bench_kernel expects a tuple of args, got {type(args).__name__}.")
    backend = get_device_backend()
    tensor_bytes = sum(a.nelement() * a.element_size() for a in args if isinstance(a, torch.Tensor))
    if args and tensor_bytes * 3 <= (1 << 30):
        pool = [tuple(a.clone() if isinstance(a, torch.Tensor) else a for a in args)
                for _ in range(3)]
    else:
        if tensor_bytes:
            _logger.warning("bench_kernel: inputs total %.2f GiB; skipping per-iteration cloning.",
                            tensor_bytes / (1 << 30))
        pool = [args]

    def run(i: int) -> Any:
        return fn(*pool[i % len(pool)])

    for i in range(n_warmup):
        backend.cache_flush()
        run(i)
    backend.synchronize()
    means = []
    for _ in range(n_trials):
        starts = [backend.Event(enable_timing=True) for _ in range(n_repeat)]
        ends = [backend.Event(enable_timing=True) for _ in range(n_repeat)]
        for i in range(n_repeat):
            backend.cache_flush()
            backend.synchronize()
            starts[i].record()
            run(i)
            ends[i].record()
        backend.synchronize()
        times = [s.elapsed_time(e) for s, e in zip(starts, ends)]
        means.append(sum(times) / len(times))
    del pool
    backend.empty_cache()
    means.sort()
    return means[len(means) // 2]


def _bench_with_mode(
    functor: Callable, args: tuple = (), mode: Optional[str] = None
) -> tuple[float, str, Optional[dict]]:
    """``(latency_ms, prof_mode, metadata)``.  ``rocprof`` falls back to
    ``events`` (with a warning) when the functor cannot be rebuilt in a child
    process or rocprofv3 is unavailable or fails; the metadata is then
    ``{"fallback_reason": ...}``.  A failed counter collection leaves the
    rocprof timing and records ``counters_error`` in its metadata."""
    mode = _prof_mode(mode)
    if mode == "rocprof":
        from tileops.benchmark.rocprof import bench_kernel_rocprof

        try:
            # one in-process call first: builds kernels and binds roofline shapes
            functor(*args)
            get_device_backend().synchronize()
            latency, _out, meta = bench_kernel_rocprof(functor, args=args)
        except (TypeError, RuntimeError, ValueError, OSError) as e:
            reason = f"{type(e).__name__}: {e}"
            _logger.warning("rocprof profiling failed (%s); falling back to events.", reason)
            return bench_kernel(functor, args=args), "events", {"fallback_reason": reason[-1000:]}
        if os.environ.get("TILEOPS_ROCPROF_COUNTERS") == "1":
            from tileops.benchmark.rocprof import bench_kernel_counters

            try:
                meta["counters"] = bench_kernel_counters(
                    functor, args=args, kernel_name=meta.get("kernel_name_resolved"))
            except (TypeError, RuntimeError, ValueError, OSError) as e:
                reason = f"{type(e).__name__}: {e}"
                _logger.warning("counter collection failed (%s)", reason)
                meta["counters_error"] = reason[-1000:]
        return latency, "rocprof", meta
    return bench_kernel(functor, args=args), "events", None


class BenchmarkBase(Generic[W], ABC):
    """Abstract benchmark of one workload: flop and byte counts plus timing."""

    def __init__(self, workload: W):
        self.workload = workload

    @abstractmethod
    def calculate_flops(self) -> Optional[float]:
        raise NotImplementedError

    @abstractmethod
    def calculate_memory(self) -> Optional[float]:
        raise NotImplementedError

    def compute_dtype(self) -> Optional[torch.dtype]:
        return getattr(self.workload, "dtype", None)

    def profile(self, functor: Any, *inputs: Any, mode: Optional[str] = None) -> dict:
        with torch.no_grad():
            latency, prof_mode, meta = _bench_with_mode(functor, args=inputs, mode=mode)
        result = self._build_result(latency)
        if meta is not None and prof_mode != "rocprof":
            result["rocprof_fallback"] = meta.get("fallback_reason")
        elif meta is not None:
            result["rocprof"] = meta
            ctr = meta.get("counters")
            if ctr:  # measured HBM traffic and MFMA busy (rocprofv3 counters)
                result["HBM bytes (counters)"] = ctr["hbm_bytes"]
                result["HBM(TB/s, counters)"] = ctr["hbm_bytes"] / (latency * 1e-3) * 1e-12
                result["MFMA busy(%)"] = ctr["mfma_busy_percent"]
        result["prof_mode"] = prof_mode
        return result

    def _build_result(self, latency: float) -> dict:
        result: dict[str, Any] = {"latency_us": latency * 1000.0}
        flops = self.calculate_flops()
        memory = self.calculate_memory()
        if flops is not None:
            result["tflops"] = flops / latency * 1e-9
        if memory is not None:
            result["bandwidth_tbs"] = memory / latency * 1e-9
        result.update(roofline_metrics(flops, memory, latency, self.compute_dtype()))
        return result


def _workload_extra_params(w: dict, shape_key: str) -> dict[str, Any]:
    reserved = WORKLOAD_RESERVED_KEYS | {shape_key}
    return {k: v for k, v in w.items()
            if isinstance(k, str) and k not in reserved and not k.startswith("__")}


def workloads_to_params(op_name: str, include_extra: bool = False) -> list:
    """pytest params ``(shape, dtype[, extra])`` of a one-input op's manifest
    workloads, with ids ``{label}-{dtype}``; unknown workload keys and a
    missing shape key raise ``KeyError``."""
    shape_key, allowed = _workload_contract(op_name)
    params = []
    for w in load_workloads(op_name):
        if shape_key not in w:
            raise KeyError(f"workload {w.get('label', w)!r} of {op_name!r} is missing {shape_key!r}.")
        unknown = sorted(repr(k) for k in w
                         if not isinstance(k, str) or (k not in allowed and not k.startswith("__")))
        if unknown:
            raise KeyError(f"workload {w.get('label', w)!r} of {op_name!r} has unknown keys {unknown}.")
        shape = tuple(w[shape_key])
        label = w.get("label", "x".join(str(s) for s in shape))
        extra = _workload_extra_params(w, shape_key) if include_extra else {}
        for dtype_str in w["dtypes"]:
            dtype = getattr(torch, dtype_str)
            values = (shape, dtype, dict(extra)) if include_extra else (shape, dtype)
            params.append(pytest.param(*values, id=f"{label}-{dtype_str}"))
    return params


class ManifestBenchmark(BenchmarkBase[Any]):
    """Benchmark whose flop / byte counts come from the Op's ``eval_roofline``
    (read after the first call, so shape-bound Ops work too)."""

    def __init__(self, op_name: str, op: Any, workload: Any):
        super().__init__(workload)
        self._op_name = op_name
        self._op = op
        self._roofline: Optional[tuple[float, float]] = None

    def _get_roofline(self) -> tuple[float, float]:
        if self._roofline is None:
            flops, nbytes = self._op.eval_roofline()
            self._roofline = (float(flops), float(nbytes))
        return self._roofline

    def calculate_flops(self) -> Optional[float]:
        return self._get_roofline()[0]

    def calculate_memory(self) -> Optional[float]:
        return self._get_roofline()[1]

    def compute_dtype(self) -> Optional[torch.dtype]:
        return getattr(self._op, "dtype", None) or super().compute_dtype()


def _extract_op_config(op: object) -> Optional[dict]:
    for holder in (op, getattr(op, "kernel", None)):
        cfg = getattr(holder, "config", None) if holder is not None else None
        if cfg:
            return cfg
    cache = getattr(op, "_kernel_cache", None)
    if cache:
        first = next(iter(cache.values()), None)
        cfg = getattr(first, "config", None)
        if cfg:
            return cfg
    return None


def _serializable(v: Any) -> bool:
    if v is None or isinstance(v, (int, float, bool, str, torch.dtype)):
        return True
    if isinstance(v, (list, tuple)):
        return all(_serializable(x) for x in v)
    if isinstance(v, dict):
        return all(isinstance(k, str) and _serializable(x) for k, x in v.items())
    return False


class BenchmarkReport:
    """Collects benchmark records; dumps a Markdown report and its JSON twin."""

    _records: dict = {}
    _prof_mode: str = DEFAULT_PROF_MODE

    @staticmethod
    def _json_safe(value: Any) -> Any:
        if value is None or isinstance(value, (bool, int, float, str)):
            return value
        if isinstance(value, torch.dtype):
            return str(value).removeprefix("torch.")
        if isinstance(value, Path):
            return str(value)
        if isinstance(value, dict):
            return {str(k): BenchmarkReport._json_safe(v)
                    for k, v in sorted(value.items(), key=lambda kv: str(kv[0]))}
        if isinstance(value, (list, tuple)):
            return [BenchmarkReport._json_safe(v) for v in value]
        return str(value)

    @staticmethod
    def _case_id(name: str, params: dict) -> str:
        """``case_id`` if given, else ``{name}-{sha256(params)[:12]}``."""
        if params.get("case_id"):
            return str(params["case_id"])
        payload = json.dumps(BenchmarkReport._json_safe(params), ensure_ascii=True,
                             sort_keys=True, separators=(",", ":"))
        return f"{name}-{hashlib.sha256(payload.encode('utf-8')).hexdigest()[:12]}"

    @staticmethod
    def _case_label(params: dict[str, Any]) -> str:
        """The workload label: explicit ``label``, else the pytest parameter
        id without its dtype suffix, else the shape, else ``N/A``."""
        if params.get("label") not in (None, ""):
            return str(params["label"])
        nodeid = os.environ.get("PYTEST_CURRENT_TEST", "").rsplit(" (", 1)[0]
        left = nodeid.rfind("[")
        if left >= 0 and nodeid.endswith("]"):
            pid = nodeid[left + 1:-1]
            dtype = params.get("dtype")
            if dtype not in (None, ""):
                suffix = f"-{str(dtype).removeprefix('torch.')}"
                if pid.endswith(suffix):
                    pid = pid[: -len(suffix)]
            if pid:
                return pid
        for key, value in params.items():
            if key == "shape" or key.endswith("_shape"):
                return "x".join(str(d) for d in value) if isinstance(value, (list, tuple)) else str(value)
        return "N/A"

    @staticmethod
    def set_prof_mode(mode: str) -> None:
        BenchmarkReport._prof_mode = mode

    @staticmethod
    def record(op_or_name, params: dict, result: dict, tag: str = "tileops") -> None:
        if isinstance(op_or_name, str):
            name, module, config = op_or_name, None, None
        else:
            name = type(op_or_name).__name__
            module = type(op_or_name).__module__
            config = _extract_op_config(op_or_name)
        kept = {k: v for k, v in params.items()
                if k not in ("test", "bm", "op", "inputs", "result") and not k.startswith("_")
                and _serializable(v)}
        kept = BenchmarkReport._json_safe(kept)
        label = BenchmarkReport._case_label(kept)
        kept.pop("label", None)
        entry = {
            "case_id": BenchmarkReport._case_id(name, kept),
            "label": label,
            "params": kept,
            "result": BenchmarkReport._json_safe(result),
            "tag": tag,
        }
        if config:
            entry["config"] = BenchmarkReport._json_safe(config)
        BenchmarkReport._records.setdefault(name, []).append(entry)
        if not hasattr(_bench_results, "entries"):
            _bench_results.entries = []
        live = {"tag": tag, "op": name, **result}
        if module:
            live["op_module"] = module
        _bench_results.entries.append(live)
        _logger.info("op=%s module=%s tag=%s latency_us=%.4f tflops=%.2f", name, module or "N/A",
                     tag, result.get("latency_us", 0), result.get("tflops", 0))

    @staticmethod
    def dump(path: Optional[str] = None) -> None:
        """Write the Markdown report (default ``TILEOPS_BENCHMARK_REPORT_PATH``
        or the session log path) and its ``.json`` companion."""
        if not BenchmarkReport._records:
            return
        path = path or os.environ.get("TILEOPS_BENCHMARK_REPORT_PATH") or profile_run_log_path(
            BenchmarkReport._prof_mode)
        out = Path(path)
        out.parent.mkdir(parents=True, exist_ok=True)
        lines = ["# MI355X Benchmark Report",
                 f"Generated: {datetime.now().strftime('%Y-%m-%d %H:%M:%S')}", "", "## Environment", ""]
        lines.extend(get_device_backend().env_metadata())
        lines.append(f"- **Profiling mode**: {BenchmarkReport._prof_mode}")
        lines.append("")
        first = ["latency_us", "Ratio(%)", "tflops", "bandwidth_tbs"]
        headers = {"latency_us": "Latency (us)", "Ratio(%)": "Ratio (%)"}
        for name, entries in BenchmarkReport._records.items():
            lines.extend([f"## {name}", ""])
            keys = list(first)
            for e in entries:
                keys.extend(k for k, v in e["result"].items()
                            if k not in keys and not isinstance(v, (dict, list)))
            by_tag: dict[str, list] = {}
            for e in entries:
                by_tag.setdefault(e["tag"], []).append(e)
            for tag, group in by_tag.items():
                lines.extend([f"### {tag}", ""])
                pkeys = list(group[0]["params"].keys())
                trailing = [k for k in ("dtype", "shape") if k in pkeys]
                pkeys = [k for k in pkeys if k not in trailing]
                has_cfg = any("config" in e for e in group)
                head = ["Label"] + [headers.get(k, k) for k in keys] + pkeys
                head += (["config"] if has_cfg else []) + trailing
                lines.append("| " + " | ".join(head) + " |")
                lines.append("| " + " | ".join(["---"] * len(head)) + " |")
                for e in group:
                    row = [str(e.get("label") or "N/A")]
                    for k in keys:
                        v = e["result"].get(k)
                        row.append("N/A" if v is None else
                                   f"{v:.4f}" if isinstance(v, (int, float)) and not isinstance(v, bool)
                                   else str(v))
                    row += [str(e["params"].get(k, "")) for k in pkeys]
                    if has_cfg:
                        row.append(str(e.get("config") or ""))
                    row += [str(e["params"].get(k, "")) for k in trailing]
                    lines.append("| " + " | ".join(row) + " |")
                lines.append("")
        out.write_text("\n".join(lines), encoding="utf-8")
        json_path = out.with_suffix(".json")
        BenchmarkReport.dump_json(str(json_path))
        print(f"\nBenchmark report saved to {out}")
        print(f"Structured benchmark report saved to {json_path}")

    @staticmethod
    def to_dict() -> dict[str, Any]:
        records = [{"operator": op, **BenchmarkReport._json_safe(e)}
                   for op, entries in BenchmarkReport._records.items() for e in entries]
        return {
            "schema_version": 1,
            "generated_at": datetime.now().astimezone().isoformat(),
            "profiling_mode_requested": BenchmarkReport._prof_mode,
            "environment": get_device_backend().env_metadata(),
            "records": records,
        }

    @staticmethod
    def dump_json(path: Optional[str] = None) -> Optional[Path]:
        if not BenchmarkReport._records:
            return None
        out = Path(path or profile_run_json_path(BenchmarkReport._prof_mode))
        out.parent.mkdir(parents=True, exist_ok=True)
        out.write_text(json.dumps(BenchmarkReport.to_dict(), indent=2, ensure_ascii=False),
                       encoding="utf-8")
        return out

    @staticmethod
    def clear() -> None:
        global _stamp
        BenchmarkReport._records.clear()
        BenchmarkReport._prof_mode = DEFAULT_PROF_MODE
        with _stamp_lock:
            _stamp = None
