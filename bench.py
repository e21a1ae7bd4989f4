"""Benchmark of the TileOPs forward-operator path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-suite] [--no-cpu-baseline]

A step is one call of the headline operator on inputs already resident in
HBM: GeluAndMulFwdOp, bf16 x[16384, 2*11008] ~ N(0,1) -> y[16384, 11008]
(the gated-GELU configuration of the benchmark spec).  Before the W warm-up
and K timed steps the operator runs untimed for 0.3 s, so that the GPU's
clocks have left their idle state.  ``value`` is its HBM
throughput in GB/s of algorithmic bytes (read x, write y).  The JSON line
also carries:

  roofline      the headline kernel's achieved / peak HBM bandwidth; the
                kernel time comes from HIP events on the launch stream over
                the timed region (one launch per step), ``traffic`` from the
                rocprofv3 FETCH_SIZE / WRITE_SIZE summary under profiles/
  cpu_baseline  the reference's own reference program of the same operator
                (its torch ``ref_program``, restated in oracle/torch_ref.py)
                on the host's CPU share, timed on a bounded sample
  suite         every other benchmark configuration (elementwise,
                predicates, FusedAddLayerNorm, LogSumExp, Argmax, MHA fwd
                causal / non-causal, GDN prefill and decode) with its own roofline
                fraction and its own CPU-baseline figure; each row runs
                untimed for 0.3 s (at least ``--warmup`` calls) before its
                ``--steps`` timed calls, so that the shader clock has
                settled under that row's own load

``--only NAME[,NAME...]`` runs just those operators (suite names, or
GeluAndMulFwdOp for the headline) and prints their entries: the form the
committed rocprofv3 summaries under profiles/ are recorded with.

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
# wall time every measured operator runs untimed before its warm-up and
# timed steps (clock settling under that operator's own load)
SUITE_WARM_S = 0.3
# rocprofv3 counter summary of the headline kernel (FETCH_SIZE / WRITE_SIZE)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gated_gelu_bf16_16384x11008_pmc.txt")


def _log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _timed(fn, args_list, steps: int, warmup: int,
           min_warm_s: float = 0.0) -> tuple[float, float]:
    """Run ``fn`` warmup + steps times (cycling through ``args_list``).

    With ``min_warm_s`` the warm-up continues (in batches of ``warmup``
    calls) until that much wall time has passed: the shader clock follows
    the board's power draw with a lag of milliseconds, so a row measured
    right after a different load (a power-limited attention run before a
    latency-bound one, or the reverse) would otherwise be timed at the
    previous load's clock.

    Returns (kernel-time ms per step from HIP events on the current stream,
    wall ms per step around the synchronised region)."""
    n = len(args_list)
    for i in range(warmup):
        fn(*args_list[i % n])
    torch.cuda.synchronize()
    t_warm, i = time.perf_counter(), warmup
    while time.perf_counter() - t_warm < min_warm_s:
        for _ in range(max(1, warmup)):
            fn(*args_list[i % n])
            i += 1
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
    # the GPU comes out of idle here: run the operator untimed for
    # SUITE_WARM_S first (memory and shader clocks ramp up under load over
    # milliseconds), then the W warm-up and K timed steps
    _timed(op, [(x,)], 1, 1, SUITE_WARM_S)
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


def cpu_threads() -> int:
    """Threads of the host's CPU share: OMP_NUM_THREADS when set (the GPU
    hosts set it to the cores a GPU is given), else the affinity mask."""
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        return int(env)
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover - non-Linux
        return os.cpu_count() or 1


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def _median_s(fn, reps: int = 3) -> float:
    """Median wall time of ``reps`` calls after one warm-up call."""
    fn()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2]


def cpu_baselines(only=None) -> dict:
    """The reference programs (oracle/torch_ref.py) on the CPU: torch's
    intra-op pool with the host's CPU share, the median of 3 runs after a
    warm-up, on a bounded sample of each benchmark workload; rates in the
    unit of the GPU figure (GB/s of algorithmic bytes, TFLOP/s)."""
    from oracle import torch_ref as tr

    threads = cpu_threads()
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(1235)
    out = {}

    def want(name):
        return only is None or name in only

    def entry(value, unit, sample):
        return {"value": round(value, 4), "unit": unit, "sample": sample}

    if want("GeluAndMulFwdOp") or want("GeluTanhAndMulFwdOp"):
        rows, n = 2048, 11008
        x = torch.randn(rows, 2 * n, generator=gen).bfloat16()
        nbytes = 3 * rows * n * 2
        for name, fn in (("GeluAndMulFwdOp", tr.gelu_and_mul),
                         ("GeluTanhAndMulFwdOp", tr.gelu_tanh_and_mul)):
            if want(name):
                t = _median_s(lambda: fn(x))
                out[name] = entry(nbytes / t / 1e9, "GB/s",
                                  f"{rows} of the 16384 rows of bf16 x[16384, 22016]")
        del x
    shape = (8192, 8192)
    n = shape[0] * shape[1]
    if any(want(k) for k in ("HardswishFwdOp", "HardsigmoidFwdOp", "ClampScalarFwdOp")):
        x = (torch.randn(shape, generator=gen) * 3).half()
        for name, fn in (("HardswishFwdOp", tr.hardswish), ("HardsigmoidFwdOp", tr.hardsigmoid),
                         ("ClampScalarFwdOp", lambda t: tr.clamp_scalar(t, -1.0, 1.0))):
            if want(name):
                t = _median_s(lambda: fn(x))
                out[name] = entry(4 * n / t / 1e9, "GB/s", "the whole fp16 x[8192, 8192]")
        del x
    if any(want(k) for k in ("IsnanFwdOp", "IsinfFwdOp", "IsfiniteFwdOp")):
        x = torch.randn(shape, generator=gen)
        idx = torch.randperm(n, generator=gen)[: n // 50]
        x.view(-1)[idx[: n // 100]] = float("inf")
        x.view(-1)[idx[n // 100:]] = float("nan")
        for name, fn in (("IsnanFwdOp", tr.isnan), ("IsinfFwdOp", tr.isinf),
                         ("IsfiniteFwdOp", tr.isfinite)):
            if want(name):
                t = _median_s(lambda: fn(x))
                out[name] = entry(5 * n / t / 1e9, "GB/s", "the whole fp32 x[8192, 8192]")
        del x
    if want("FusedAddLayerNormFwdOp"):
        rows, hid = 4096, 4096
        x = torch.randn(rows, hid, generator=gen).bfloat16()
        r = torch.randn(rows, hid, generator=gen).bfloat16()
        w = 1 + 0.1 * torch.randn(hid, generator=gen)
        b = 0.1 * torch.randn(hid, generator=gen)
        t = _median_s(lambda: tr.fused_add_layer_norm(x, r, w, b, 1e-5))
        out["FusedAddLayerNormFwdOp"] = entry((4 * rows * hid * 2 + 2 * hid * 4) / t / 1e9,
                                              "GB/s", f"{rows} of the 32768 rows")
        del x, r
    if want("LogSumExpFwdOp") or want("ArgmaxFwdOp"):
        rows, cols = 8192, 4096
        x = torch.randn(rows, cols, generator=gen) * 2.0
        if want("LogSumExpFwdOp"):
            t = _median_s(lambda: tr.logsumexp(x))
            out["LogSumExpFwdOp"] = entry((rows * cols + rows) * 4 / t / 1e9, "GB/s",
                                          f"{rows} of the 32768 rows")
        if want("ArgmaxFwdOp"):
            t = _median_s(lambda: tr.argmax(x))
            out["ArgmaxFwdOp"] = entry((rows * cols * 4 + rows * 8) / t / 1e9, "GB/s",
                                       f"{rows} of the 32768 rows")
        del x
    for causal in (False, True):
        name = f"MultiHeadAttentionFwdOp[causal={causal}]"
        if not want(name) and not want("MultiHeadAttentionFwdOp"):
            continue
        S, D, heads = 4096, 128, 2
        q, k, v = (torch.randn(1, S, heads, D, generator=gen).bfloat16() for _ in range(3))
        t = _median_s(lambda: tr.mha_fwd(q, k, v, causal), reps=1)
        flops = 4 * heads * S * S * D / (2 if causal else 1)
        out[name] = entry(flops / t / 1e12, "TFLOP/s",
                          f"{heads} of the 256 (batch, head) pairs (SDPA in fp32); the rate "
                          "holds for all 256, which are independent")
    if want("GatedDeltaNetPrefillFwdOp"):
        # the whole workload: the token recurrence takes about a second here
        B, T, H, K = 4, 8192, 16, 128
        q = F_normalize(torch.randn(B, T, H, K, generator=gen)).bfloat16()
        k = F_normalize(torch.randn(B, T, H, K, generator=gen)).bfloat16()
        v = torch.randn(B, T, H, K, generator=gen).bfloat16()
        g = torch.nn.functional.logsigmoid(torch.randn(B, T, H, generator=gen))
        beta = torch.sigmoid(torch.randn(B, T, H, generator=gen))
        t = _median_s(lambda: tr.gdn_sequential(q, k, v, g, beta, K**-0.5))
        C = 64
        flops = (6 * C * C * K + 4 * C * C * K + 6 * C * K * K + C**3 // 3) * (T // C) * B * H
        out["GatedDeltaNetPrefillFwdOp"] = entry(
            flops / t / 1e12, "TFLOP/s",
            f"the whole workload (B4 T8192 H16, every token), {t:.2f} s per run, counted "
            "with the chunked-form flops")
        del q, k, v
    if want("GatedDeltaNetDecodeFwdOp"):
        B, H, K = 16, 32, 128
        q = F_normalize(torch.randn(B, 1, H, K, generator=gen)).bfloat16()
        k = F_normalize(torch.randn(B, 1, H, K, generator=gen)).bfloat16()
        v = torch.randn(B, 1, H, K, generator=gen).bfloat16()
        g = torch.nn.functional.logsigmoid(torch.randn(B, 1, H, generator=gen))
        beta = torch.sigmoid(torch.randn(B, 1, H, generator=gen))
        h0 = torch.randn(B, H, K, K, generator=gen)
        t = _median_s(lambda: tr.gdn_sequential(q, k, v, g, beta, K**-0.5, h0))
        nbytes = B * H * (8 * K * K + 4 * K * 2 + 8)
        out["GatedDeltaNetDecodeFwdOp"] = entry(nbytes / t / 1e9, "GB/s",
                                                f"{B} of the 256 sequences (the token "
                                                "recurrence on one token)")
    cores = {"threads": threads, "host_cpus": os.cpu_count(), "cpu": _cpu_model()}
    for v in out.values():
        v.update(cores)
    return out


def F_normalize(x: torch.Tensor) -> torch.Tensor:
    return torch.nn.functional.normalize(x, dim=-1)


# ---------------------------------------------------------------------------
# suite: the other benchmark configurations
# ---------------------------------------------------------------------------
def _mem_entry(name, op, args_list, nbytes, steps, warmup, workload):
    ms, _ = _timed(op, args_list, steps, warmup, SUITE_WARM_S)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return name, {
        "workload": workload,
        "us": round(ms * 1e3, 2),
        "GB/s": round(gbs, 1),
        "frac": round(gbs / HBM_PEAK_GBS, 4),
        "bound": "hbm",
    }


def _mfma_entry(name, op, args_list, flops, steps, warmup, workload):
    ms, _ = _timed(op, args_list, steps, warmup, SUITE_WARM_S)
    tf = flops / (ms * 1e-3) / 1e12
    return name, {
        "workload": workload,
        "ms": round(ms, 4),
        "TFLOP/s": round(tf, 1),
        "frac": round(tf / BF16_PEAK_TFLOPS, 4),
        "bound": "mfma",
    }


def bench_suite(steps: int, warmup: int, only=None) -> dict:
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

    def want(*names):
        return only is None or any(nm in only for nm in names)

    # elementwise family, fp16 [8192, 8192] ~ N(0, 3^2)
    shape = (8192, 8192)
    n = shape[0] * shape[1]
    unary = ("HardswishFwdOp", "HardsigmoidFwdOp", "ClampScalarFwdOp")
    if want(*unary):
        rot = _rotations(4 * n)
        xs = [ScaledNormalWorkload(shape, torch.float16, 3.0).gen_inputs() for _ in range(rot)]
        for name, op in (
            ("HardswishFwdOp", HardswishFwdOp(n, torch.float16)),
            ("HardsigmoidFwdOp", HardsigmoidFwdOp(n, torch.float16)),
            ("ClampScalarFwdOp", ClampScalarFwdOp(n, torch.float16, min=-1.0, max=1.0)),
        ):
            if want(name):
                k, v = _mem_entry(name, op, xs, op.eval_roofline()[1], steps, warmup,
                                  "fp16 x[8192, 8192] ~ N(0, 9)")
                out[k] = v
                _log(f"{k}: {v}")
        del xs

    # predicates, fp32 [8192, 8192], 1% +-inf and 1% NaN at random positions
    preds = ("IsnanFwdOp", "IsinfFwdOp", "IsfiniteFwdOp")
    if want(*preds):
        rot = _rotations(5 * n)
        xs = [ScatteredSpecialWorkload(shape, torch.float32).gen_inputs() for _ in range(rot)]
        for name, op in (
            ("IsnanFwdOp", IsnanFwdOp(n, torch.float32)),
            ("IsinfFwdOp", IsinfFwdOp(n, torch.float32)),
            ("IsfiniteFwdOp", IsfiniteFwdOp(n, torch.float32)),
        ):
            if want(name):
                k, v = _mem_entry(name, op, xs, op.eval_roofline()[1], steps, warmup,
                                  "fp32 x[8192, 8192], 1% +-inf, 1% NaN")
                out[k] = v
                _log(f"{k}: {v}")
        del xs

    # GeluTanhAndMul, same shape as the headline
    if want("GeluTanhAndMulFwdOp"):
        M, N = 16384, 11008
        x = torch.randn(M, 2 * N, device=dev, dtype=torch.bfloat16)
        op = GeluTanhAndMulFwdOp(M, N, torch.bfloat16)
        k, v = _mem_entry("GeluTanhAndMulFwdOp", op, [(x,)], op.eval_roofline()[1], steps,
                          warmup, "bf16 x[16384, 22016] ~ N(0, 1)")
        out[k] = v
        _log(f"{k}: {v}")
        del x

    # FusedAddLayerNorm, bf16 [32768, 4096], fp32 gamma / beta
    if want("FusedAddLayerNormFwdOp"):
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
    if want("LogSumExpFwdOp", "ArgmaxFwdOp"):
        x = torch.randn(32768, 4096, device=dev) * 2.0
        for name, op in (("LogSumExpFwdOp", LogSumExpFwdOp(dtype=torch.float32, dim=-1)),
                         ("ArgmaxFwdOp", ArgmaxFwdOp(dtype=torch.float32, dim=-1))):
            if want(name):
                op(x)
                k, v = _mem_entry(name, op, [(x,)], op.eval_roofline()[1], steps, warmup,
                                  "fp32 x[32768, 4096] ~ N(0, 4), dim=-1")
                out[k] = v
                _log(f"{k}: {v}")
        del x

    # MHA forward, bf16 BSHD (8, 4096, 32, 128)
    mha = ("MultiHeadAttentionFwdOp[causal=False]", "MultiHeadAttentionFwdOp[causal=True]")
    if want("MultiHeadAttentionFwdOp", *mha):
        B, S, H, D = 8, 4096, 32, 128
        q, kk, vv = (torch.randn(B, S, H, D, device=dev, dtype=torch.bfloat16) for _ in range(3))
        for causal in (False, True):
            name = f"MultiHeadAttentionFwdOp[causal={causal}]"
            if not want(name, "MultiHeadAttentionFwdOp"):
                continue
            op = MultiHeadAttentionFwdOp(B, H, S, D, causal, torch.bfloat16)
            # at least 3 warm-up and 10 timed launches (~2 ms each): fewer
            # are timed while the clocks are still settling
            k, v = _mfma_entry(name, op, [(q, kk, vv)], op.eval_roofline()[0],
                               max(10, steps // 2), max(3, warmup),
                               "bf16 q, k, v (8, 4096, 32, 128) BSHD, scale 1/sqrt(128)")
            out[k] = v
            _log(f"{k}: {v}")
        del q, kk, vv

    # GDN decode: one token for a serving batch, bf16 q, k, v, fp32 state
    if want("GatedDeltaNetDecodeFwdOp"):
        from tileops.ops.linear_attention import GatedDeltaNetDecodeFwdOp
        from tileops.workloads.linear_attention import GdnDecodeWorkload

        B, H, K, V = 256, 32, 128, 128
        inputs = GdnDecodeWorkload(B, H, K, V, torch.bfloat16).gen_inputs()
        op = GatedDeltaNetDecodeFwdOp(B, H, K, V)
        op(*inputs)
        k, v = _mem_entry("GatedDeltaNetDecodeFwdOp", op, [inputs], op.eval_roofline()[1], steps,
                          warmup, "one token of 256 sequences x 32 heads: bf16 q, k "
                          "(L2-normalised) [256, 32, 128], v [256, 32, 128]; fp32 g, beta; "
                          "fp32 state [256, 32, 128, 128] read and a new one written")
        out[k] = v
        _log(f"{k}: {v}")
        del inputs

    if not want("GatedDeltaNetPrefillFwdOp"):
        return out
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
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-suite", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", help="comma-separated operators to run (profiling); prints "
                    "their entries only")
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
    only = set(args.only.split(",")) if args.only else None
    with contextlib.redirect_stdout(sys.stderr):
        if only is not None:
            res = {}
            if "GeluAndMulFwdOp" in only:
                h = bench_headline(args.steps, args.warmup)
                res["GeluAndMulFwdOp"] = {"us": round(h["kernel_ms"] * 1e3, 2),
                                          "GB/s": round(h["gbs"], 1),
                                          "frac": round(h["gbs"] / HBM_PEAK_GBS, 4)}
            res.update(bench_suite(args.steps, args.warmup, only))
            if not args.no_cpu_baseline:
                for name, c in cpu_baselines(only).items():
                    res.setdefault(name, {})["cpu"] = c
        else:
            head = bench_headline(args.steps, args.warmup)
            _log(f"headline GeluAndMulFwdOp: {head['gbs']:.1f} GB/s, "
                 f"{head['kernel_ms'] * 1e3:.1f} us")
            suite = {} if args.no_suite else bench_suite(args.steps, args.warmup)
            cpus = {} if args.no_cpu_baseline else cpu_baselines(
                None if not args.no_suite else {"GeluAndMulFwdOp"})
            for name, c in cpus.items():
                if name in suite:
                    suite[name]["cpu"] = c
            hc = cpus.get("GeluAndMulFwdOp")
            cpu = None if hc is None else {
                "value": hc["value"], "unit": hc["unit"], "cores": hc["threads"],
                "kind": "port",
                "sample": f"the reference's reference program (torch, "
                f"tests/ops/test_gelu_and_mul.py:63-77, restated in oracle/torch_ref.py) on "
                f"{hc['sample']}, median of 3 runs after a warm-up, {hc['threads']} threads "
                f"of a {hc['host_cpus']}-CPU host ({hc['cpu']})",
            }
    if only is not None:
        print(json.dumps({"only": sorted(only), "results": res}), flush=True)
        return 0

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
