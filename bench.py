"""Benchmark of the TileOPs forward-operator path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-suite] [--no-cpu-baseline]

A step is one call of the headline operator on inputs already resident in
HBM: GeluAndMulFwdOp, bf16 x[16384, 2*11008] ~ N(0,1) -> y[16384, 11008]
(the gated-GELU configuration of the benchmark spec).  ``value`` is its HBM
throughput in GB/s of algorithmic bytes (read x, write y).  The JSON line
also carries:

  roofline      the headline kernel's achieved / peak HBM bandwidth; the
                kernel time comes from HIP events on the launch stream over
                the timed region (one launch per step), ``traffic`` from the
                rocprofv3 FETCH_SIZE / WRITE_SIZE summary under profiles/
  cpu_baseline  the CPU oracle of the same operator on the host, one core
  suite         every other benchmark configuration (elementwise,
                predicates, FusedAddLayerNorm, LogSumExp, Argmax, MHA fwd
                causal / non-causal, GDN prefill) with its own roofline
                fraction

Only one GPU is used; ``--gpus`` above 1 exits with an explanation.
"""

from __future__ import annotations

import argparse
import contextlib
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "tile-ascendnpu-ops_amd"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, TFLOP/s
METRIC = "HBM GB/s (% peak) for eltwise/norm ops; bf16 TFLOP/s (% MFMA) MHA fwd, GDN"
# rocprofv3 counter summary of the headline kernel (FETCH_SIZE / WRITE_SIZE)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gated_gelu_bf16_16384x11008_pmc.txt")


def _log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _timed(fn, args_list, steps: int, warmup: int) -> tuple[float, float]:
    """Run ``fn`` warmup + steps times (cycling through ``args_list``).

    Returns (kernel-time ms per step from HIP events on the current stream,
    wall ms per step around the synchronised region)."""
    n = len(args_list)
    for i in range(warmup):
        fn(*args_list[i % n])
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for i in range(steps):
        fn(*args_list[i % n])
    end.record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return start.elapsed_time(end) / steps, wall


def _rotations(nbytes_per_set: int) -> int:
    """Input sets to cycle so the working set exceeds the 256 MB Infinity Cache 4x."""
    return max(1, min(8, -(-(1 << 30) // max(nbytes_per_set, 1))))


def _read_traffic() -> int | None:
    try:
        with open(TRAFFIC_FILE) as f:
            m = re.search(r"traffic_bytes_per_launch:\s*([0-9]+)", f.read())
        return int(m.group(1)) if m else None
    except OSError:
        return None


# ---------------------------------------------------------------------------
# headline
# ---------------------------------------------------------------------------
def bench_headline(steps: int, warmup: int) -> dict:
    from tileops.ops.elementwise import GeluAndMulFwdOp

    M, N = 16384, 11008
    torch.manual_seed(1235)
    x = torch.randn(M, 2 * N, device="cuda", dtype=torch.bfloat16)
    op = GeluAndMulFwdOp(M, N, torch.bfloat16)
    _, nbytes = op.eval_roofline()
    kern_ms, wall_ms = _timed(op, [(x,)], steps, warmup)
    gbs = nbytes / (kern_ms * 1e-3) / 1e9
    return {
        "kernel_ms": kern_ms,
        "wall_ms": wall_ms,
        "bytes": nbytes,
        "gbs": gbs,
        "M": M,
        "N": N,
    }


def cpu_baseline_gelu(M: int, N: int) -> dict:
    """The CPU oracle of GeluAndMul (numpy + scipy erf, one thread) over the
    whole workload in 2048-row chunks; GB/s of the same algorithmic bytes."""
    import numpy as np

    from oracle import tileops_oracle as orc

    rng = np.random.default_rng(1235)
    chunk = 2048
    elapsed = 0.0
    rows = 0
    for r0 in range(0, M, chunk):
        x = orc.round_to("bfloat16", rng.standard_normal((chunk, 2 * N), dtype=np.float32))
        t0 = time.perf_counter()
        orc.gelu_and_mul(x, "bfloat16")
        elapsed += time.perf_counter() - t0
        rows += chunk
    nbytes = 3 * rows * N * 2
    return {
        "value": round(nbytes / elapsed / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"full workload, {rows} rows of bf16 x[*, {2 * N}] in {chunk}-row chunks "
        f"({elapsed:.1f} s, numpy/scipy oracle, single thread; host has "
        f"{os.cpu_count()} cores)",
    }


# ---------------------------------------------------------------------------
# suite: the other benchmark configurations
# ---------------------------------------------------------------------------
def _mem_entry(name, op, args_list, nbytes, steps, warmup, workload):
    ms, _ = _timed(op, args_list, steps, warmup)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return name, {
        "workload": workload,
        "us": round(ms * 1e3, 2),
        "GB/s": round(gbs, 1),
        "frac": round(gbs / HBM_PEAK_GBS, 4),
        "bound": "hbm",
    }


def _mfma_entry(name, op, args_list, flops, steps, warmup, workload):
    ms, _ = _timed(op, args_list, steps, warmup)
    tf = flops / (ms * 1e-3) / 1e12
    return name, {
        "workload": workload,
        "ms": round(ms, 4),
        "TFLOP/s": round(tf, 1),
        "frac": round(tf / BF16_PEAK_TFLOPS, 4),
        "bound": "mfma",
    }


def bench_suite(steps: int, warmup: int) -> dict:
    from tileops.ops.attention import MultiHeadAttentionFwdOp
    from tileops.ops.elementwise import (
        ClampScalarFwdOp,
        GeluTanhAndMulFwdOp,
        HardsigmoidFwdOp,
        HardswishFwdOp,
        IsfiniteFwdOp,
        IsinfFwdOp,
        IsnanFwdOp,
    )
    from tileops.ops.norm import FusedAddLayerNormFwdOp
    from tileops.ops.reduction import ArgmaxFwdOp, LogSumExpFwdOp
    from tileops.workloads.elementwise import ScaledNormalWorkload, ScatteredSpecialWorkload
    from tileops.workloads.norm import FusedAddLayerNormWorkload

    out = {}
    torch.manual_seed(1235)
    dev = "cuda"

    # elementwise family, fp16 [8192, 8192] ~ N(0, 3^2)
    shape = (8192, 8192)
    n = shape[0] * shape[1]
    rot = _rotations(4 * n)
    xs = [ScaledNormalWorkload(shape, torch.float16, 3.0).gen_inputs() for _ in range(rot)]
    for name, op in (
        ("HardswishFwdOp", HardswishFwdOp(n, torch.float16)),
        ("HardsigmoidFwdOp", HardsigmoidFwdOp(n, torch.float16)),
        ("ClampScalarFwdOp", ClampScalarFwdOp(n, torch.float16, min=-1.0, max=1.0)),
    ):
        k, v = _mem_entry(name, op, xs, op.eval_roofline()[1], steps, warmup,
                          "fp16 x[8192, 8192] ~ N(0, 9)")
        out[k] = v
        _log(f"{k}: {v}")
    del xs

    # predicates, fp32 [8192, 8192], 1% +-inf and 1% NaN at random positions
    rot = _rotations(5 * n)
    xs = [ScatteredSpecialWorkload(shape, torch.float32).gen_inputs() for _ in range(rot)]
    for name, op in (
        ("IsnanFwdOp", IsnanFwdOp(n, torch.float32)),
        ("IsinfFwdOp", IsinfFwdOp(n, torch.float32)),
        ("IsfiniteFwdOp", IsfiniteFwdOp(n, torch.float32)),
    ):
        k, v = _mem_entry(name, op, xs, op.eval_roofline()[1], steps, warmup,
                          "fp32 x[8192, 8192], 1% +-inf, 1% NaN")
        out[k] = v
        _log(f"{k}: {v}")
    del xs

    # GeluTanhAndMul, same shape as the headline
    M, N = 16384, 11008
    x = torch.randn(M, 2 * N, device=dev, dtype=torch.bfloat16)
    op = GeluTanhAndMulFwdOp(M, N, torch.bfloat16)
    k, v = _mem_entry("GeluTanhAndMulFwdOp", op, [(x,)], op.eval_roofline()[1], steps, warmup,
                      "bf16 x[16384, 22016] ~ N(0, 1)")
    out[k] = v
    _log(f"{k}: {v}")
    del x

    # FusedAddLayerNorm, bf16 [32768, 4096], fp32 gamma / beta
    wl = FusedAddLayerNormWorkload(32768, 4096, torch.bfloat16, param_dtype=torch.float32)
    inputs = wl.gen_inputs()
    op = FusedAddLayerNormFwdOp(dtype=torch.bfloat16, eps=1e-5)
    op(*inputs)
    k, v = _mem_entry("FusedAddLayerNormFwdOp", op, [inputs], op.eval_roofline()[1], steps,
                      warmup, "bf16 x, residual [32768, 4096]; fp32 gamma ~ N(1, 0.01), "
                      "beta ~ N(0, 0.01); eps 1e-5")
    out[k] = v
    _log(f"{k}: {v}")
    del inputs

    # LogSumExp / Argmax, fp32 [32768, 4096] ~ N(0, 4)
    x = torch.randn(32768, 4096, device=dev) * 2.0
    for name, op in (("LogSumExpFwdOp", LogSumExpFwdOp(dtype=torch.float32, dim=-1)),
                     ("ArgmaxFwdOp", ArgmaxFwdOp(dtype=torch.float32, dim=-1))):
        op(x)
        k, v = _mem_entry(name, op, [(x,)], op.eval_roofline()[1], steps, warmup,
                          "fp32 x[32768, 4096] ~ N(0, 4), dim=-1")
        out[k] = v
        _log(f"{k}: {v}")
    del x

    # MHA forward, bf16 BSHD (8, 4096, 32, 128)
    B, S, H, D = 8, 4096, 32, 128
    q, kk, vv = (torch.randn(B, S, H, D, device=dev, dtype=torch.bfloat16) for _ in range(3))
    for causal in (False, True):
        op = MultiHeadAttentionFwdOp(B, H, S, D, causal, torch.bfloat16)
        name = f"MultiHeadAttentionFwdOp[causal={causal}]"
        k, v = _mfma_entry(name, op, [(q, kk, vv)], op.eval_roofline()[0], max(3, steps // 4),
                           max(1, warmup // 2), "bf16 q, k, v (8, 4096, 32, 128) BSHD, "
                           "scale 1/sqrt(128)")
        out[k] = v
        _log(f"{k}: {v}")
    del q, kk, vv

    try:
        from tileops.ops.linear_attention import GatedDeltaNetPrefillFwdOp
        from tileops.workloads.linear_attention import GdnPrefillWorkload

        wl = GdnPrefillWorkload(4, 8192, 16, 128, 128, torch.bfloat16)
        inputs = wl.gen_inputs()
        op = GatedDeltaNetPrefillFwdOp(4, 8192, 16, 128, 128, chunk_size=64)
        flops, nbytes = op.eval_roofline()
        k, v = _mfma_entry("GatedDeltaNetPrefillFwdOp", op, [inputs], flops, steps, warmup,
                           "bf16 q, k (L2-normalised), v [4, 8192, 16, 128]; fp32 g, beta; "
                           "chunk 64, zero initial state")
        v["GB/s"] = round(nbytes / (v["ms"] * 1e-3) / 1e9, 1)
        out[k] = v
        _log(f"{k}: {v}")
    except (ImportError, RuntimeError) as e:  # GDN op not built yet
        out["GatedDeltaNetPrefillFwdOp"] = {"status": f"not measured: {e}"}
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-suite", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 1 GiB device copy (counter calibration for "
                    "rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(
            "bench.py measures one GPU: every operator here is single-device (across GPUs "
            "its rows / heads would be sharded with no exchange); run with --gpus 1.",
            file=sys.stderr,
        )
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1

    if args.calibrate_copy:
        src = torch.empty(1 << 29, dtype=torch.int16, device="cuda")  # 1 GiB
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "copy", "bytes_read": 1 << 30, "bytes_written": 1 << 30,
                          "launches": args.steps}))
        return 0

    # stdout carries the one JSON line only: everything the operators print
    # while they are built and run goes to stderr
    with contextlib.redirect_stdout(sys.stderr):
        head = bench_headline(args.steps, args.warmup)
        _log(f"headline GeluAndMulFwdOp: {head['gbs']:.1f} GB/s, {head['kernel_ms'] * 1e3:.1f} us")
        suite = {} if args.no_suite else bench_suite(args.steps, args.warmup)
        cpu = None if args.no_cpu_baseline else cpu_baseline_gelu(head["M"], head["N"])

    line = {
        "metric": METRIC,
        "value": round(head["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["wall_ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "GeluAndMulFwdOp: bf16 x[16384, 2*11008] ~ N(0,1) (gate | value) -> "
            "y[16384, 11008], fp32 math",
            "op": "GeluAndMulFwdOp",
            "rows": head["M"],
            "cols": head["N"],
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(head["gbs"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(head["gbs"] / HBM_PEAK_GBS, 4),
            "traffic": _read_traffic(),
            "kernel_us": round(head["kernel_ms"] * 1e3, 2),
            "algorithmic_bytes": head["bytes"],
        },
        "cpu_baseline": cpu,
        "suite": suite,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
