"""Board power and shader clock of one MI355X under sustained attention and GEMM load.

Runs, for about six seconds each, the attention forward (bf16 (8, 4096,
32, 128), non-causal and causal) and the vendor bf16 GEMM (torch.matmul,
16384^3), while a child process samples ``amd-smi metric -p -c`` (socket
power, GFX clock) about three times a second.  Prints, per phase, the
time per call, the throughput and the mean power and clock of the samples
taken inside the phase.  Under this load the board sits at its power limit
and the clock is what gives: the throughput of a kernel is then set by the
energy it spends per flop, and the vendor GEMM under the same limit is the
practical ceiling for any bf16 MFMA kernel.

    python tile-ascendnpu-ops_amd/benchmarks/power_clock.py [--secs 6]
"""

import argparse
import os
import re
import subprocess
import sys
import tempfile
import time


def _start_sampler(path: str, count: int) -> subprocess.Popen:
    # started before anything touches the GPU, as a child process
    script = (
        f"for i in $(seq 1 {count}); do echo \"T $(date +%s.%N)\"; "
        "timeout 5 amd-smi metric -p -c -g 0 2>&1; sleep 0.25; done"
    )
    out = open(path, "w")
    return subprocess.Popen(["bash", "-c", script], stdout=out, stderr=subprocess.STDOUT)


def _parse_samples(path: str):
    rows, cur = [], None
    with open(path) as f:
        for line in f:
            if line.startswith("T "):
                if cur is not None:
                    rows.append(cur)
                cur = {"t": float(line.split()[1])}
            elif cur is not None and "SOCKET_POWER" in line:
                m = re.search(r"(\d+(?:\.\d+)?) W", line)
                if m:
                    cur["power"] = float(m.group(1))
            elif cur is not None and "clk" not in cur and re.match(r"\s+CLK: \d", line):
                cur["clk"] = float(re.search(r"(\d+) MHz", line).group(1))
    if cur is not None:
        rows.append(cur)
    return rows


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--secs", type=float, default=6.0, help="seconds per phase")
    args = ap.parse_args()

    log = os.path.join(tempfile.gettempdir(), f"power_clock_{os.getpid()}.log")
    sampler = _start_sampler(log, int(8 * args.secs) + 60)

    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import torch

    from tileops.ops.attention import MultiHeadAttentionFwdOp

    dev = torch.device("cuda:0")
    B, H, S, D = 8, 32, 4096, 128
    q = torch.randn(B, S, H, D, dtype=torch.bfloat16, device=dev)
    k = torch.randn_like(q)
    v = torch.randn_like(q)
    ops = {c: MultiHeadAttentionFwdOp(B, H, S, D, c, torch.bfloat16) for c in (False, True)}
    n = 16384
    a = torch.randn(n, n, dtype=torch.bfloat16, device=dev)
    b = torch.randn_like(a)
    for c in (False, True):
        ops[c](q, k, v)
    torch.matmul(a, b)
    torch.cuda.synchronize()

    mha_flops = 4.0 * B * H * S * S * D
    phases = []

    def phase(name, fn, flops):
        t0 = time.time()
        calls = 0
        while time.time() - t0 < args.secs:
            for _ in range(4):
                fn()
            torch.cuda.synchronize()
            calls += 4
        t1 = time.time()
        phases.append((name, t0, t1, (t1 - t0) / calls, flops))
        print(f"phase {name}: {calls} calls", file=sys.stderr, flush=True)
        time.sleep(1.5)

    time.sleep(2.0)
    phases.append(("idle", time.time() - 2.0, time.time(), None, None))
    phase("attention bf16 (8,4096,32,128) non-causal", lambda: ops[False](q, k, v), mha_flops)
    phase("attention bf16 (8,4096,32,128) causal", lambda: ops[True](q, k, v), mha_flops / 2)
    phase("vendor GEMM bf16 16384^3 (torch.matmul)", lambda: torch.matmul(a, b), 2.0 * n ** 3)
    time.sleep(1.0)
    sampler.terminate()
    sampler.wait(timeout=10)

    rows = _parse_samples(log)
    print(f"{'phase':44s} {'ms/call':>9s} {'TFLOP/s':>9s} {'% of 2.5P':>9s} "
          f"{'power W':>8s} {'GFX MHz':>8s} {'TFLOP/s per kW':>15s}  samples")
    for name, t0, t1, sec, flops in phases:
        # samples inside the phase, skipping its first second (the power
        # controller settles within it)
        inside = [r for r in rows if t0 + 1.0 <= r["t"] <= t1 and "power" in r and "clk" in r]
        pw = sum(r["power"] for r in inside) / len(inside) if inside else float("nan")
        clk = sum(r["clk"] for r in inside) / len(inside) if inside else float("nan")
        if sec is None:
            print(f"{name:44s} {'':>9s} {'':>9s} {'':>9s} {pw:8.0f} {clk:8.0f} {'':>15s}  {len(inside)}")
            continue
        tf = flops / sec / 1e12
        print(f"{name:44s} {sec * 1e3:9.3f} {tf:9.1f} {tf / 25.0:8.1f}% {pw:8.0f} {clk:8.0f} "
              f"{tf / pw * 1e3:15.1f}  {len(inside)}")
    os.remove(log)
    return 0


if __name__ == "__main__":
    sys.exit(main())
