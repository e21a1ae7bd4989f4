from tileops.workloads.workload_base import (
    FixtureBase,
    FixtureMeta,
    RandnWorkload,
    WorkloadBase,
)

__all__ = ["FixtureBase", "FixtureMeta", "RandnWorkload", "WorkloadBase"]
