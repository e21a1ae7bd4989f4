"""TileOPs forward operators on AMD Instinct MI355X (gfx950).

Layer structure (kept from the reference TileOPs package, so callers switch
without code changes):

    manifest  -- spec source of truth (YAML): signatures, workloads, roofline
    workloads -- seeded input generation
    ops       -- Op classes: validation, reshape, kernel dispatch, roofline
    kernels   -- Kernel classes: each forwards into libtileops_hip.so, the
                 C-ABI library of hand-written HIP kernels for gfx950
    testing   -- TestBase: correctness against a reference program
    benchmark -- latency / bandwidth / TFLOP/s measurement (HIP events,
                 rocprofv3)
    reporting -- the ``tileops-report`` CLI

All device-specific code goes through :mod:`tileops.device`.
"""

from tileops.device import get_device_backend

__all__ = ["get_device_backend"]
