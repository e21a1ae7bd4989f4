"""Op base class: validation, kernel dispatch and roofline of one operator.

Interface kept from the reference (examples/TileOPs/tileops/ops/op_base.py:31-130):
``default_kernel_map`` / ``dispatch_kernel`` / ``kernel_map`` injection,
``forward`` + ``__call__``, ``eval_roofline() -> (flops, bytes)`` and the
``_cache_key`` helper.  Architecture checks compare a Kernel's
``supported_archs`` with the device's ISA name (``gfx950``) or marketing name.
"""

from __future__ import annotations

import warnings
from abc import ABC, abstractmethod
from typing import Hashable, Optional, Union

import torch

from tileops.device import HIPBackend, get_device_backend
from tileops.kernels.kernel_base import Kernel


class Op(ABC):
    """Base class for TileOPs operators."""

    kernel: Optional[Kernel] = None
    kernel_map: Optional[dict[str, Kernel]] = None
    dtype: Optional[torch.dtype] = None
    input_shapes: Optional[list[tuple]] = None
    _static_axes: frozenset[tuple[int, int]] = frozenset()

    @property
    @abstractmethod
    def default_kernel_map(self) -> dict[str, Kernel]:
        raise NotImplementedError("Op must implement default_kernel_map")

    def _install_kernel_map(self, candidate_map: Optional[dict[str, Kernel]] = None) -> None:
        default_map = self.default_kernel_map
        if default_map is None or len(default_map) == 0:
            self.kernel_map = dict(candidate_map) if candidate_map else {}
            return
        resolved: dict[str, Kernel] = {}
        backend = get_device_backend()
        for name, default_kernel in default_map.items():
            kernel_type = (
                candidate_map[name]
                if candidate_map is not None and name in candidate_map
                else default_kernel
            )
            if (
                kernel_type is not None
                and kernel_type.supported_archs is not None
                and not _arch_supported(kernel_type.supported_archs, backend)
            ):
                raise ValueError(
                    f"{kernel_type.__name__} is not supported on backend "
                    f"{backend.name} (supported: {kernel_type.supported_archs})"
                )
            resolved[name] = kernel_type
        self.kernel_map = resolved

    def dispatch_kernel(self, kernel_map: Optional[dict[str, Kernel]] = None) -> None:
        self._install_kernel_map(kernel_map)

    @abstractmethod
    def forward(self, *args: object, **kwargs: object) -> Union[torch.Tensor, tuple]:
        raise NotImplementedError("forward method is not implemented")

    def __call__(self, *args: object, **kwargs: object) -> Union[torch.Tensor, tuple]:
        return self.forward(*args, **kwargs)

    def eval_roofline(self) -> tuple[int, int]:
        raise NotImplementedError(
            f"{type(self).__name__}.eval_roofline() must be implemented by the concrete Op."
        )

    def _cache_key(self, *input_shapes: tuple[int, ...]) -> Hashable:
        if not self._static_axes and type(self)._cache_key is Op._cache_key:
            warnings.warn(
                f"{type(self).__name__}: Op._cache_key() called with empty _static_axes "
                f"and no subclass override.",
                stacklevel=2,
            )
        return tuple(
            s
            for i, shape in enumerate(input_shapes)
            for axis, s in enumerate(shape)
            if (i, axis) not in self._static_axes
        )


def _arch_supported(supported: Optional[list], backend: object) -> bool:
    """True when the current device's ISA name (``gfx950:sramecc+:xnack-``
    style) or marketing name contains a listed arch.  With no GPU (the host
    backend) there is nothing to compare against: Ops can still be built (shapes, rooflines)
    and any launch fails on its own for want of a device tensor."""
    if supported is None or not backend.is_available() or not isinstance(backend, HIPBackend):
        return True
    dev = backend.current_device()
    names = [backend.get_device_name(dev)]
    arch = getattr(backend, "arch_name", None)
    if arch is not None:
        names.append(arch(dev))
    return any(str(a) in n for a in supported for n in names if n)
