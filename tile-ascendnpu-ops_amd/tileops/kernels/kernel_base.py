"""Kernel base class: the Python face of one HIP kernel family.

Interface kept from the reference (examples/TileOPs/tileops/kernels/kernel_base.py:22-94):
``supported_archs``, ``default_config`` / ``init_config`` (which prints the
resolved config), ``dtype_str``, and ``__call__`` -> ``forward``.  A concrete
Kernel's ``forward`` allocates its outputs with PyTorch and launches the
gfx950 kernels through libtileops_hip.so on the tensors' current stream.

``default_config`` states the launch shape compiled into the device code.
Keys listed in ``tunable_config`` are passed to the launch; any other key,
or a value that differs from the compiled one, raises ``ValueError`` rather
than being ignored.  ``check_tensor`` is the input check every ``forward``
runs before launching: the device code trusts the sizes it is given, so a
tensor of another dtype or size must never reach it.
"""

from abc import ABC, abstractmethod
from typing import Any, Dict, Optional, Sequence

import torch

# Every kernel of libtileops_hip.so is compiled for this ISA only.
GFX950 = ["gfx950"]


class Kernel(ABC):
    """Abstract base class for the HIP-backed operator kernels.

    Subclasses set ``supported_archs`` (ISA names such as ``"gfx950"``;
    ``None`` means no restriction) and ``default_config``.
    """

    dtype: Optional[torch.dtype] = None
    config: Dict[str, Any]
    supported_archs: Optional[list] = GFX950
    kernel: Optional[Any] = None
    # Regular expression matching the (mangled) names of every device kernel
    # one forward call launches; the rocprofv3 benchmark path sums the
    # kernel-trace rows it matches.
    profile_kernel_name: str = ""
    # config keys whose values reach the launch (all others are compiled in)
    tunable_config: tuple = ()

    def __init__(self, *args: Any, **kwargs: Any) -> None:
        self.config = {}

    def init_config(self, config: Optional[Dict[str, Any]] = None) -> None:
        merged = dict(self.default_config)
        if config is not None:
            name = self.__class__.__name__
            unknown = sorted(set(config) - set(merged))
            if unknown:
                raise ValueError(
                    f"{name}: unknown config keys {unknown}; supported: {sorted(merged)}")
            for k, v in config.items():
                if v is None:
                    continue
                if k not in self.tunable_config and v != merged[k]:
                    raise ValueError(
                        f"{name}: config {k}={v!r} is not available; the compiled kernel "
                        f"uses {k}={merged[k]!r}")
                merged[k] = v
        self.config = merged
        print(f"{self.__class__.__name__} initialized with config: {self.config}")

    def check_tensor(self, name: str, t: torch.Tensor, dtype: Optional[torch.dtype] = None,
                     shape: Optional[Sequence[int]] = None,
                     numel: Optional[int] = None) -> None:
        """Raise ``ValueError`` unless ``t`` has the dtype, shape or element
        count this kernel was built for."""
        cls = self.__class__.__name__
        if dtype is not None and t.dtype != dtype:
            raise ValueError(f"{cls}: expected {name}.dtype {dtype}, got {t.dtype}")
        if shape is not None and tuple(t.shape) != tuple(shape):
            raise ValueError(
                f"{cls}: expected {name}.shape {tuple(shape)}, got {tuple(t.shape)}")
        if numel is not None and t.numel() != numel:
            raise ValueError(f"{cls}: expected {numel} elements in {name}, got {t.numel()}")

    @property
    def dtype_str(self) -> str:
        return self.dtype_to_str(self.dtype)

    @staticmethod
    def dtype_to_str(dtype: torch.dtype) -> str:
        return str(dtype).split(".")[-1]

    @property
    def default_config(self) -> Dict[str, Any]:
        return {}

    @abstractmethod
    def forward(self, *args: Any, **kwargs: Any) -> Any:
        raise NotImplementedError

    def __call__(self, *args: Any, **kwargs: Any) -> Any:
        return self.forward(*args, **kwargs)
