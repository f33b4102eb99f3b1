"""CPU baseline for bench.py: the reference's own path for one Linear layer, timed on the host.
TEST INFRASTRUCTURE ONLY (imported by bench.py's cpu_baseline leg, never by the product).

The reference runs every projection as a bf16 `nn.Linear` → `F.linear(x, W)` (bias=False,
torch/nn/modules/linear.py:134), on the CPU when no GPU is present
(src/llm_serving_engine/model/model_runner.py:49, 184-200). This module times exactly that
call on the same shapes and input distributions as the GPU workload and reports it in the
GPU metric's unit: algorithmic bytes of the int8 layer (K·N + 4N + 2MK + 2MN) per second.
"""

from __future__ import annotations

import os
import platform
import time

import torch


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def time_bf16_linear_sweep(
    shapes: list[tuple[int, int]], ms: list[int], budget_s: float = 15.0, seed: int = 1000
) -> dict:
    """Median-of-repeats time of `F.linear(x, W_bf16)` over every (K, N) x M case, on all cores
    this process may use. Returns bytes/s in the int8 layer's algorithmic bytes."""
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(seed)
    total_bytes = 0
    total_s = 0.0
    per_case = []
    deadline = time.perf_counter() + budget_s
    for k, n in shapes:
        w = (torch.randn(n, k, generator=gen) * 0.02).to(torch.bfloat16)
        for m in ms:
            x = torch.randn(m, k, generator=gen).to(torch.bfloat16)
            torch.nn.functional.linear(x, w)  # warm-up
            times = []
            for _ in range(5):
                t0 = time.perf_counter_ns()
                torch.nn.functional.linear(x, w)
                times.append(time.perf_counter_ns() - t0)
                if time.perf_counter() > deadline and len(times) >= 2:
                    break
            t = sorted(times)[len(times) // 2] / 1e9
            b = k * n + 4 * n + 2 * m * k + 2 * m * n
            per_case.append({"k": k, "n": n, "m": m, "s": t})
            total_bytes += b
            total_s += t
        del w
    return {
        "bytes": total_bytes,
        "seconds": total_s,
        "gbps": total_bytes / total_s / 1e9,
        "threads": threads,
        "cpu": cpu_model(),
        "cases": per_case,
    }
