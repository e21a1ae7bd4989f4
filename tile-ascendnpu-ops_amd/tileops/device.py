"""Device backend for MI355X: one HIP device layer behind the reference API.

Every device-specific operation (detection, synchronisation, events, the
cache flush used by benchmarks, device properties, environment metadata)
goes through :class:`DeviceBackend`, as in the reference
(examples/TileOPs/tileops/device.py:37-103).  Two implementations exist:

- :class:`HIPBackend` -- PyTorch-ROCm.  PyTorch exposes HIP devices under the
  ``"cuda"`` device type, so ``name`` is ``"cuda"`` and workloads that build
  tensors with ``device=get_device_backend().name`` land in HBM.
- :class:`CPUBackend` -- no GPU present (build / unit-test hosts).  Ops refuse
  to run on it: every kernel launches HIP code only.
"""

from __future__ import annotations

import subprocess
from abc import ABC, abstractmethod
from typing import Optional

import torch

__all__ = [
    "DEFAULT_DEVICE",
    "CPUBackend",
    "DeviceBackend",
    "HIPBackend",
    "get_device_backend",
    "reset_device_backend",
]

# MI355X: 256 MB of Infinity Cache (MALL) sits in front of HBM; a flush
# buffer of twice that evicts every line a benchmark iteration left behind.
_MALL_BYTES = 256 * 1024 * 1024
_FLUSH_BYTES = 2 * _MALL_BYTES


class DeviceBackend(ABC):
    """Abstract device backend (the reference's adaptation surface)."""

    name: str = "abstract"

    @abstractmethod
    def is_available(self) -> bool: ...

    @abstractmethod
    def device_count(self) -> int: ...

    @abstractmethod
    def current_device(self) -> int: ...

    @abstractmethod
    def synchronize(self, device: Optional[int] = None) -> None: ...

    @abstractmethod
    def empty_cache(self) -> None: ...

    @abstractmethod
    def get_device_name(self, device: Optional[int] = None) -> str: ...

    @abstractmethod
    def get_device_properties(self, device: Optional[int] = None) -> object: ...

    @abstractmethod
    def is_device_tensor(self, tensor: torch.Tensor) -> bool: ...

    @abstractmethod
    def Event(self, enable_timing: bool = False) -> object: ...

    @abstractmethod
    def manual_seed_all(self, seed: int) -> None: ...

    @abstractmethod
    def env_metadata(self) -> list[str]:
        """Markdown lines describing the device environment."""

    def cache_flush(self) -> None:
        """Evict device caches before a timed benchmark iteration (no-op here)."""
        return

    def supports_profiler(self) -> bool:
        return False

    def shared_memory_budget(self, device: Optional[int] = None) -> int:
        """On-chip scratch budget in bytes for tile sizing."""
        return 48 * 1024

    def arch_name(self, device: Optional[int] = None) -> str:
        """ISA name of the device (e.g. ``gfx950``); empty when unknown."""
        return ""


class HIPBackend(DeviceBackend):
    """AMD GPU backend through PyTorch-ROCm (HIP streams, events, allocator)."""

    name = "cuda"  # PyTorch's device type for HIP devices

    def is_available(self) -> bool:
        return torch.cuda.is_available() and torch.version.hip is not None

    def device_count(self) -> int:
        return torch.cuda.device_count()

    def current_device(self) -> int:
        return torch.cuda.current_device()

    def synchronize(self, device: Optional[int] = None) -> None:
        torch.cuda.synchronize(device)

    def empty_cache(self) -> None:
        torch.cuda.empty_cache()

    def get_device_name(self, device: Optional[int] = None) -> str:
        return torch.cuda.get_device_name(device)

    def get_device_properties(self, device: Optional[int] = None) -> object:
        return torch.cuda.get_device_properties(
            torch.cuda.current_device() if device is None else device
        )

    def arch_name(self, device: Optional[int] = None) -> str:
        props = self.get_device_properties(device)
        return str(getattr(props, "gcnArchName", "")).split(":")[0]

    def is_device_tensor(self, tensor: torch.Tensor) -> bool:
        return tensor.is_cuda

    def Event(self, enable_timing: bool = False) -> object:
        return torch.cuda.Event(enable_timing=enable_timing)

    def manual_seed_all(self, seed: int) -> None:
        torch.cuda.manual_seed_all(seed)

    def supports_profiler(self) -> bool:
        return True

    def shared_memory_budget(self, device: Optional[int] = None) -> int:
        """LDS bytes one workgroup may allocate (160 KiB on gfx950)."""
        props = self.get_device_properties(device)
        for attr in ("shared_memory_per_block_optin", "shared_memory_per_block"):
            v = int(getattr(props, attr, 0) or 0)
            if v > 0:
                return v
        return 64 * 1024

    _flush_buf: Optional[torch.Tensor] = None

    def cache_flush(self) -> None:
        """Overwrite twice the Infinity Cache so the next kernel reads HBM."""
        if self._flush_buf is None:
            self._flush_buf = torch.empty(_FLUSH_BYTES // 4, dtype=torch.int32, device="cuda")
        self._flush_buf.zero_()

    def env_metadata(self) -> list[str]:
        lines = [
            f"- **Torch version**: {torch.__version__}",
            f"- **HIP version (torch)**: {torch.version.hip or 'N/A'}",
        ]
        if self.is_available():
            lines.append(f"- **GPU model**: {self.get_device_name(0)} ({self.arch_name(0)})")
            lines.append(f"- **GPU count**: {self.device_count()}")
        else:
            lines.append("- **GPU model**: N/A (no HIP device)")
        smi = _query_rocm_smi()
        if smi:
            lines.append(f"- **rocm-smi**: {smi}")
        return lines


def _query_rocm_smi() -> str:
    try:
        r = subprocess.run(
            ["rocm-smi", "--showproductname", "--json"],
            capture_output=True,
            text=True,
            timeout=5,
        )
        return r.stdout.strip().replace("\n", " ")[:200] if r.returncode == 0 else ""
    except (FileNotFoundError, subprocess.TimeoutExpired):
        return ""


class CPUBackend(DeviceBackend):
    """Host-only backend: shapes, validation and roofline work; kernels do not."""

    name = "cpu"

    def is_available(self) -> bool:
        return True

    def device_count(self) -> int:
        return 1

    def current_device(self) -> int:
        return 0

    def synchronize(self, device: Optional[int] = None) -> None:
        pass

    def empty_cache(self) -> None:
        pass

    def get_device_name(self, device: Optional[int] = None) -> str:
        return "CPU"

    def get_device_properties(self, device: Optional[int] = None) -> object:
        class _CPUProps:
            name = "CPU"
            total_memory = 0

        return _CPUProps()

    def is_device_tensor(self, tensor: torch.Tensor) -> bool:
        return tensor.device.type == "cpu"

    def Event(self, enable_timing: bool = False) -> object:
        class _CPUEvent:
            def record(self, stream=None) -> None:
                import time

                self._t = time.perf_counter()

            def synchronize(self) -> None:
                pass

            def elapsed_time(self, other: "_CPUEvent") -> float:
                return (other._t - self._t) * 1000.0

        return _CPUEvent()

    def manual_seed_all(self, seed: int) -> None:
        torch.manual_seed(seed)

    def env_metadata(self) -> list[str]:
        return [f"- **Torch version**: {torch.__version__}", "- **Device**: CPU (no accelerator)"]


def _detect_backend() -> DeviceBackend:
    hip = HIPBackend()
    if hip.is_available():
        return hip
    return CPUBackend()


_backend: Optional[DeviceBackend] = None


def get_device_backend() -> DeviceBackend:
    """Return the process-wide :class:`DeviceBackend`."""
    global _backend
    if _backend is None:
        _backend = _detect_backend()
    return _backend


def reset_device_backend() -> None:
    """Drop the cached backend (tests)."""
    global _backend
    _backend = None


DEFAULT_DEVICE: str = get_device_backend().name
