"""CPU baseline for bench.py: the reference's own path for one Linear layer, timed on the host.
TEST INFRASTRUCTURE ONLY (imported by bench.py's cpu_baseline leg, never by the product).

The reference runs every projection as a bf16 `nn.Linear` → `F.linear(x, W)` (bias=False,
torch/nn/modules/linear.py:134), on the CPU when no GPU is present
(src/llm_serving_engine/model/model_runner.py:49, 184-200). This module times exactly that
call on the same shapes and input distributions as the GPU workload and reports it in the
GPU metric's unit: algorithmic bytes of the int8 layer (K·N + 4N + 2MK + 2MN) per second.
Beside it, `time_int8_restatements` times torch's own int8 CPU kernels for the same layer:
`aten._weight_int8pack_mm` (W8A16) and per-token quantization + `torch._int_mm` + the epilogue
(W8A8), in the same unit.
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


def time_int8_restatements(
    shapes: list[tuple[int, int]], ms: list[int], budget_s: float = 10.0, seed: int = 1001
) -> dict:
    """Median-of-repeats time of torch's int8 CPU kernels over every (K, N) x M case: W8A16 as
    `aten._weight_int8pack_mm(x, q, s)` (bf16 x and scales), W8A8 as per-token quantization of
    x, `torch._int_mm(xq, q^T)` and the fp32 epilogue. Each is reported as the int8 layer's
    algorithmic bytes per second (the GPU metric's unit), with `budget_s` seconds per mode."""
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(seed)

    def w8a16(x, q, s_bf16, s32):
        return torch.ops.aten._weight_int8pack_mm(x, q, s_bf16)

    def w8a8(x, q, s_bf16, s32):
        xf = x.float()
        sx = xf.abs().amax(dim=1, keepdim=True) / 127.0
        sx = torch.where(sx > 0, sx, torch.ones_like(sx))
        xq = torch.clamp(torch.round(xf / sx), -127, 127).to(torch.int8)
        acc = torch._int_mm(xq, q.t())
        return ((acc.float() * sx) * s32).to(torch.bfloat16)

    out = {"threads": threads, "cpu": cpu_model()}
    cases = []
    for k, n in shapes:
        q = torch.randint(-127, 128, (n, k), generator=gen, dtype=torch.int8)
        s32 = torch.rand(n, generator=gen) * 1e-3 + 1e-4
        for m in ms:
            x = torch.randn(m, k, generator=gen).to(torch.bfloat16)
            cases.append((k, n, m, x, q, s32))
    for name, fn in (("w8a16_weight_int8pack_mm", w8a16), ("w8a8_int_mm", w8a8)):
        total_bytes = 0
        total_s = 0.0
        deadline = time.perf_counter() + budget_s
        for k, n, m, x, q, s32 in cases:
            s_bf16 = s32.to(torch.bfloat16)
            fn(x, q, s_bf16, s32)  # warm-up
            times = []
            for _ in range(5):
                t0 = time.perf_counter_ns()
                fn(x, q, s_bf16, s32)
                times.append(time.perf_counter_ns() - t0)
                if time.perf_counter() > deadline and len(times) >= 2:
                    break
            total_s += sorted(times)[len(times) // 2] / 1e9
            total_bytes += k * n + 4 * n + 2 * m * k + 2 * m * n
        out[name] = {"gbps": total_bytes / total_s / 1e9, "seconds": total_s}
    return out
