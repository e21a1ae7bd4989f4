"""rocprofv3 kernel-time measurement of an Op rebuilt in a subprocess.

The subprocess reconstructs the Op from its constructor-named attributes
(the contract of the reference's examples/TileOPs/tileops/benchmark/msprof.py:108-139),
so Ops keep every ``__init__`` argument as an attribute of the same name.
"""

from __future__ import annotations

import inspect
from typing import Any

import torch

__all__ = ["_extract_op_init_args"]


def _is_serializable(val: Any) -> bool:
    if val is None or isinstance(val, (bool, int, float, str, torch.dtype)):
        return True
    if isinstance(val, (list, tuple)):
        return all(_is_serializable(v) for v in val)
    return False


def _extract_op_init_args(op: Any) -> dict:
    """Constructor arguments of ``op`` read back from its attributes.

    Walks ``type(op).__init__``'s named parameters and keeps those the
    instance holds under the same name with a plain serializable value
    (kernels, kernel maps and caches are skipped)."""
    try:
        sig = inspect.signature(type(op).__init__)
    except (TypeError, ValueError):
        return {}
    out: dict = {}
    for name, param in sig.parameters.items():
        if name == "self" or param.kind in (param.VAR_POSITIONAL, param.VAR_KEYWORD):
            continue
        if hasattr(op, name):
            val = getattr(op, name)
            if _is_serializable(val):
                out[name] = val
    return out


# ---------------------------------------------------------------------------
# rocprofv3 result databases (rocpd SQLite, the default output of rocprofv3)
# ---------------------------------------------------------------------------
def read_kernel_stats(db_path: str, name_filter: str = "") -> list[dict]:
    """Per-kernel dispatch statistics from a ``rocprofv3 --kernel-trace`` database.

    Returns one dict per kernel name (sorted by total time): ``name``,
    ``calls``, ``avg_us``, ``min_us``, ``max_us``, ``total_us``."""
    import sqlite3

    con = sqlite3.connect(db_path)
    try:
        rows = con.execute(
            "select name, count(*), avg(end - start), min(end - start), max(end - start), "
            "sum(end - start) from kernels where name like ? group by name "
            "order by sum(end - start) desc",
            (f"%{name_filter}%",),
        ).fetchall()
    finally:
        con.close()
    return [
        {
            "name": r[0],
            "calls": int(r[1]),
            "avg_us": r[2] / 1e3,
            "min_us": r[3] / 1e3,
            "max_us": r[4] / 1e3,
            "total_us": r[5] / 1e3,
        }
        for r in rows
    ]


def read_counters(db_path: str, name_filter: str = "") -> list[dict]:
    """Per-kernel averages of every counter in a ``rocprofv3 --pmc`` database."""
    import sqlite3

    con = sqlite3.connect(db_path)
    try:
        rows = con.execute(
            "select kernel_name, counter_name, count(*), avg(value), min(value), max(value) "
            "from counters_collection where kernel_name like ? "
            "group by kernel_name, counter_name",
            (f"%{name_filter}%",),
        ).fetchall()
    finally:
        con.close()
    return [
        {"kernel": r[0], "counter": r[1], "dispatches": int(r[2]), "avg": r[3], "min": r[4],
         "max": r[5]}
        for r in rows
    ]


def _first(rows: list[dict], counter: str) -> float:
    for r in rows:
        if r["counter"] == counter:
            return r["avg"]
    raise KeyError(counter)


def hbm_traffic(kernel_fetch_db: str, kernel_write_db: str, copy_fetch_db: str,
                copy_write_db: str, kernel_filter: str, copy_bytes: int) -> dict:
    """HBM bytes per launch of one kernel from FETCH_SIZE / WRITE_SIZE (KiB per
    dispatch), each scaled by what the same counter reads for a plain device
    copy of ``copy_bytes`` bytes read and written."""
    kf = _first(read_counters(kernel_fetch_db, kernel_filter), "FETCH_SIZE")
    kw = _first(read_counters(kernel_write_db, kernel_filter), "WRITE_SIZE")
    cf = _first(read_counters(copy_fetch_db, "copy"), "FETCH_SIZE")
    cw = _first(read_counters(copy_write_db, "copy"), "WRITE_SIZE")
    f_scale = copy_bytes / (cf * 1024.0)
    w_scale = copy_bytes / (cw * 1024.0)
    read_b = kf * 1024.0 * f_scale
    write_b = kw * 1024.0 * w_scale
    return {
        "fetch_kib": kf,
        "write_kib": kw,
        "copy_fetch_kib": cf,
        "copy_write_kib": cw,
        "fetch_scale": f_scale,
        "write_scale": w_scale,
        "read_bytes": int(round(read_b)),
        "write_bytes": int(round(write_b)),
        "traffic_bytes_per_launch": int(round(read_b + write_b)),
    }


def _main(argv=None) -> int:
    import argparse
    import json

    ap = argparse.ArgumentParser(prog="python -m tileops.benchmark.rocprof",
                                 description="Summaries of rocprofv3 result databases")
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats", help="kernel-trace statistics")
    s.add_argument("db")
    s.add_argument("--filter", default="")
    t = sub.add_parser("traffic", help="calibrated HBM traffic of one kernel")
    t.add_argument("kernel_fetch_db")
    t.add_argument("kernel_write_db")
    t.add_argument("copy_fetch_db")
    t.add_argument("copy_write_db")
    t.add_argument("--filter", required=True)
    t.add_argument("--copy-bytes", type=int, default=1 << 30)
    args = ap.parse_args(argv)
    if args.cmd == "stats":
        print(f"{'calls':>6} {'avg_us':>10} {'min_us':>10} {'max_us':>10}  kernel")
        for r in read_kernel_stats(args.db, args.filter):
            print(f"{r['calls']:6d} {r['avg_us']:10.2f} {r['min_us']:10.2f} {r['max_us']:10.2f}"
                  f"  {r['name'][:110]}")
    else:
        res = hbm_traffic(args.kernel_fetch_db, args.kernel_write_db, args.copy_fetch_db,
                          args.copy_write_db, args.filter, args.copy_bytes)
        for k, v in res.items():
            print(f"{k}: {v}")
        print(json.dumps(res))
    return 0


if __name__ == "__main__":
    raise SystemExit(_main())
