"""Sustained bf16 MFMA throughput of one MI355X through the vendor GEMM.

``torch.matmul`` on bf16 square matrices (hipBLASLt on ROCm), timed with
HIP events after warm-up: the practical ceiling that any bf16 MFMA kernel
on this GPU (the attention forward included) can be compared with, since
under sustained matrix-core load the shader clock sits well below the
2.4 GHz that the 2.5 PFLOP/s dense bf16 figure assumes.

    python tile-ascendnpu-ops_amd/benchmarks/gemm_ceiling.py
"""

import torch

PEAK_TFLOPS = 2500.0  # MI355X dense bf16


def main() -> None:
    for n, iters in ((8192, 20), (16384, 5)):
        a = torch.randn(n, n, device="cuda", dtype=torch.bfloat16)
        b = torch.randn(n, n, device="cuda", dtype=torch.bfloat16)
        for _ in range(3):
            a @ b
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(iters):
            a @ b
        end.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / iters
        tflops = 2 * n**3 / ms / 1e9
        print(f"bf16 GEMM {n}x{n}x{n}: {ms:.3f} ms  {tflops:.1f} TFLOP/s  "
              f"{100 * tflops / PEAK_TFLOPS:.1f}% of {PEAK_TFLOPS:.0f}", flush=True)


if __name__ == "__main__":
    main()
