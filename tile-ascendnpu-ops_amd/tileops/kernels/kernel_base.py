"""Kernel base class: the Python face of one HIP kernel family.

Interface kept from the reference (examples/TileOPs/tileops/kernels/kernel_base.py:22-94):
``supported_archs``, ``default_config`` / ``init_config`` (which prints the
resolved config), ``dtype_str``, and ``__call__`` -> ``forward``.  A concrete
Kernel's ``forward`` allocates its outputs with PyTorch and launches the
gfx950 kernels through libtileops_hip.so on the tensors' current stream.
"""

from abc import ABC, abstractmethod
from typing import Any, Dict, Optional

import torch


class Kernel(ABC):
    """Abstract base class for the HIP-backed operator kernels.

    Subclasses set ``supported_archs`` (ISA names such as ``"gfx950"``;
    ``None`` means no restriction) and ``default_config``.
    """

    dtype: Optional[torch.dtype] = None
    config: Dict[str, Any]
    supported_archs: Optional[list] = None
    kernel: Optional[Any] = None
    # Name of the dominant device kernel (a substring of the HIP symbol), used
    # by the rocprofv3 benchmark path to filter kernel-trace rows.
    profile_kernel_name: str = ""

    def __init__(self, *args: Any, **kwargs: Any) -> None:
        self.config = {}

    def init_config(self, config: Optional[Dict[str, Any]] = None) -> None:
        if config is not None:
            merged = dict(self.default_config)
            for k in merged:
                if config.get(k) is not None:
                    merged[k] = config[k]
            self.config = merged
        else:
            self.config = dict(self.default_config)
        print(f"{self.__class__.__name__} initialized with config: {self.config}")

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
