"""Small helpers shared by the harness (reference: tileops/utils/utils.py:5)."""

import torch

_DTYPES = {
    "float32": torch.float32,
    "fp32": torch.float32,
    "float": torch.float32,
    "float16": torch.float16,
    "fp16": torch.float16,
    "half": torch.float16,
    "bfloat16": torch.bfloat16,
    "bf16": torch.bfloat16,
    "int64": torch.int64,
    "int32": torch.int32,
    "bool": torch.bool,
}


def str2dtype(name: str) -> torch.dtype:
    """Map a manifest dtype string (``"float16"``, ``"bf16"`` ...) to a torch dtype."""
    key = str(name).strip().replace("torch.", "")
    if key not in _DTYPES:
        raise ValueError(f"unknown dtype string {name!r}")
    return _DTYPES[key]
