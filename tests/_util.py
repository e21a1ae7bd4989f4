"""Helpers shared by the GPU parity tests: tensor <-> oracle conversion and
the reference suite's tolerance tables."""

import numpy as np
import torch

NAMES = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16"}


def to_np(t: torch.Tensor) -> np.ndarray:
    """Device tensor -> float32 numpy (bool / int tensors keep their dtype)."""
    t = t.detach().cpu()
    if t.dtype in (torch.bool, torch.int64, torch.int32):
        return t.numpy()
    return t.float().numpy()


def from_np(a: np.ndarray, like: torch.Tensor, dtype: torch.dtype = None) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype or like.dtype).to(like.device)


def ref_tolerance(dtype: torch.dtype) -> tuple[float, float]:
    """(atol, rtol) of the reference tests (e.g. tests/ops/test_hardswish.py:18-24)."""
    if dtype == torch.float32:
        return 1e-5, 1e-5
    if dtype == torch.float16:
        return 1e-3, 1e-3
    return 1.6e-2, 1.6e-2


# rtol = atol = 1e-2 for half-precision outputs at the benchmark configs
HALF_PRECISION_TOL = 1e-2


def assert_close_np(got: np.ndarray, ref: np.ndarray, atol: float, rtol: float, what: str = ""):
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} vs {ref.shape}"
    nan_g, nan_r = np.isnan(got), np.isnan(ref)
    assert (nan_g == nan_r).all(), f"{what}: NaN mismatch at {np.argwhere(nan_g != nan_r)[:5]}"
    ok = ~nan_r
    inf_r = np.isinf(ref) & ok
    assert (got[inf_r] == ref[inf_r]).all(), f"{what}: inf mismatch"
    fin = ok & ~inf_r
    err = np.abs(got[fin] - ref[fin])
    bound = atol + rtol * np.abs(ref[fin])
    bad = err > bound
    if bad.any():
        idx = np.argwhere(fin)[np.argmax(err - bound)]
        raise AssertionError(
            f"{what}: {bad.sum()} / {fin.sum()} elements out of tolerance "
            f"(atol={atol}, rtol={rtol}); worst at {tuple(idx)}: got "
            f"{got[tuple(idx)]} ref {ref[tuple(idx)]}; max abs err {err.max():.3e}"
        )


def assert_bits_equal(got: np.ndarray, ref: np.ndarray, what: str = ""):
    """Bit-identical float arrays, except that any NaN matches any NaN."""
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    ng, nr = np.isnan(got), np.isnan(ref)
    assert np.array_equal(ng, nr), f"{what}: NaN positions differ"
    g, r = got[~ng].view(np.uint32), ref[~nr].view(np.uint32)
    bad = np.nonzero(g != r)[0]
    assert bad.size == 0, (
        f"{what}: {bad.size} values differ, first got {got[~ng][bad[:4]]} ref {ref[~nr][bad[:4]]}"
    )
