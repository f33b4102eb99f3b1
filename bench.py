"""Benchmark of the int8 quantized Linear forward on one MI355X.

Headline (`value`): config 1, the W8A16 decode sweep. One step runs the decode path (the decode
kernel; for gate_up at 64 tokens a 64 x 128 tile of the tiled kernel) over the
four Llama-3-8B linear shapes (K, N) in {(4096, 6144) fused QKV, (4096, 4096) o_proj,
(4096, 28672) fused gate_up, (14336, 4096) down} at M in {1, 8, 32, 64}, over LAYERS distinct
copies of the weights (LAYERS x 218 MB, far beyond the 256 MB Infinity Cache, so every launch
streams its weights from HBM). value = algorithmic bytes (K·N + 4N + 2MK + 2MN per launch) /
time, in GB/s.

Secondary figures on the same line: config 2 (W8A16 prefill GEMM, TFLOP/s at M=2048 and the
M sweep), config 3 (W8A8 quantize + int8 GEMM, TOP/s) and the fused gate_up + SiLU-mul kernels
(decode GB/s, prefill TFLOP/s, each beside the unfused GEMM + SiLU-mul they replace), plus the
roofline of the decode kernel and the CPU baseline (the reference's bf16 F.linear on the host
cores).

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--no-secondary]

Profiling (the decode sweep alone, then a CPU-side summary of the rocprofv3 output):

    rocprofv3 --kernel-trace --stats -d T -o run --output-format csv -- \
        python3 bench.py --only decode --steps 5 --warmup 2
    rocprofv3 --pmc FETCH_SIZE -d F -o run --output-format csv -- \
        python3 bench.py --only decode --steps 1 --warmup 0
    rocprofv3 --pmc WRITE_SIZE -d W -o run --output-format csv -- \
        python3 bench.py --only decode --steps 1 --warmup 0
    python3 bench.py --summarize-profiles T F W

`--only decode` first runs one plain 64 MiB elementwise copy (int32 bitwise_not: 64 MiB read,
64 MiB written), whose FETCH_SIZE and WRITE_SIZE readings scale the counters to bytes.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import sys
from pathlib import Path

REPO_ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO_ROOT))

HBM_PEAK_GBPS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
INT8_PEAK_TOPS = 5000.0
SHAPES = [(4096, 6144), (4096, 4096), (4096, 28672), (14336, 4096)]  # (K, N)
SHAPE_NAMES = ["qkv", "o_proj", "gate_up", "down"]
KV_SHAPE = (4096, 1024)  # (K, N) of the separate k_proj and v_proj the drop-in runs
DECODE_MS = [1, 8, 32, 64]
PREFILL_MS = [512, 2048, 8192]
W8A8_MS = [1, 32, 512, 4096]
LAYERS = 8
CALIBRATION_BYTES = 64 << 20
PROFILE_MD = REPO_ROOT / "profiles" / "skinny_kernel_decode_sweep.md"
PROFILE_TRAFFIC = REPO_ROOT / "profiles" / "skinny_kernel_decode_sweep.traffic.json"
CSRC = REPO_ROOT / "llm-serving-engine_amd" / "csrc"
PROFILE_PREFILL = REPO_ROOT / "profiles" / "tiled_gemm_kernel_prefill.md"
PROFILE_W8A8 = REPO_ROOT / "profiles" / "tiled_gemm_kernel_w8a8.md"
PROFILE_GLU = REPO_ROOT / "profiles" / "fused_gate_up_kernels.md"
PROFILE_ATTN = REPO_ROOT / "profiles" / "paged_attn_kernel_decode.md"
PROFILE_HEAD = REPO_ROOT / "profiles" / "bf16_lm_head_kernels.md"
PROFILE_STEP = REPO_ROOT / "profiles" / "decode_step_kernels.md"
CUS, SIMDS_PER_CU, XCDS = 256, 4, 8


def decode_bytes(m: int, k: int, n: int) -> int:
    return k * n + 4 * n + 2 * m * k + 2 * m * n


def parse() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-secondary", action="store_true", help="skip prefill and W8A8 figures")
    p.add_argument("--only", choices=["decode", "prefill", "w8a8", "glu", "attention",
                                      "lm-head", "decode-step", "decode-step-linears", "tp8",
                                      "mid"],
                   help="one family; decode-step is config 4 (a 32-layer model's decode step)")
    p.add_argument("--summarize-profiles", nargs=3, metavar=("TRACE", "FETCH", "WRITE"),
                   help="summarize rocprofv3 output dirs of the decode sweep into profiles/")
    p.add_argument("--summarize-attention", metavar="TRACE",
                   help="write the paged attention profile summary from a kernel trace of "
                        "--only attention")
    p.add_argument("--summarize-lm-head", metavar="TRACE",
                   help="write the packed bf16 lm_head profile summary from a kernel trace of "
                        "--only lm-head --steps 5")
    p.add_argument("--summarize-glu", metavar="TRACE",
                   help="write the fused gate_up profile summary from a kernel trace of --only glu")
    p.add_argument("--summarize-w8a8", nargs=2, metavar=("TRACE", "PMC"),
                   help="summarize rocprofv3 output dirs of --only w8a8 into profiles/")
    p.add_argument("--summarize-decode-step", metavar="TRACE",
                   help="write the config-4 per-kernel summary from a kernel trace of "
                        "--only decode-step-linears")
    p.add_argument("--summarize-prefill", nargs=2, metavar=("TRACE", "PMC"),
                   help="summarize rocprofv3 output dirs of --only prefill into profiles/")
    return p.parse_args()


def make_weights(pkg, dev, k: int, n: int, copies: int, gen):
    """`copies` independent (packed q, s) pairs, quantized and packed on the GPU from
    W ~ N(0, 0.02)."""
    import torch

    out = []
    for _ in range(copies):
        w = (torch.randn(n, k, generator=gen, device="cpu") * 0.02).to(dev)
        q, s = pkg.ops.quantize_weight_per_channel(w)
        out.append((pkg.ops.pack_weight(q), s))
        del w, q
    return out


def time_region(fn, steps: int, warmup: int) -> float:
    """Seconds for exactly `steps` calls of fn, between HIP events on the current stream and
    device synchronisations on both sides, after `warmup` untimed calls."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / 1e3


def calibration_copy(dev) -> None:
    """One plain elementwise copy of CALIBRATION_BYTES (int32 bitwise_not), the reference reading
    for the FETCH_SIZE / WRITE_SIZE counters."""
    import torch

    src = torch.ones(CALIBRATION_BYTES // 4, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    torch.bitwise_not(src, out=dst)
    torch.cuda.synchronize()
    del src, dst


def bench_decode(pkg, dev, steps: int, warmup: int, gen) -> dict:
    import torch

    weights = [make_weights(pkg, dev, k, n, LAYERS, gen) for k, n in SHAPES]
    xs = {(m, k): torch.randn(m, k, generator=gen).to(torch.bfloat16).to(dev)
          for m in DECODE_MS for k in {k for k, _ in SHAPES}}
    outs = {(m, n): torch.empty(m, n, dtype=torch.bfloat16, device=dev)
            for m in DECODE_MS for _, n in SHAPES}
    # Raw C-ABI launches (m, k, n, args without the stream), replayed from a captured graph so
    # the timed region measures the kernels, not host-side launch cost.
    # The launches run in order on one stream, so they share one workspace of the largest size.
    lib = pkg.library()
    ws_bytes = max(lib.lse_workspace_bytes(0, m, n, k) for m in DECODE_MS
                   for k, n in SHAPES + [KV_SHAPE])
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
    calls = []
    for m in DECODE_MS:
        for layer in range(LAYERS):
            for si, (k, n) in enumerate(SHAPES):
                q, s = weights[si][layer]
                calls.append((m, k, n, (xs[(m, k)].data_ptr(), k, q.data_ptr(), s.data_ptr(),
                                        outs[(m, n)].data_ptr(), n, m, n, k, 1, ws.data_ptr(),
                                        ws_bytes)))
    fn_ptr = pkg.library().lse_w8a16_gemm_algo

    def graph_of(sub):
        def launch():
            stream = torch.cuda.current_stream().cuda_stream
            for *_, args in sub:
                st = fn_ptr(*args, stream)
                if st:
                    raise RuntimeError(f"lse_w8a16_gemm_algo status {st}")

        launch()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            launch()
        return g

    step = graph_of(calls).replay
    total_bytes = LAYERS * sum(decode_bytes(m, k, n) for m in DECODE_MS for k, n in SHAPES)
    seconds = time_region(step, steps, warmup)
    per_step = seconds / steps

    # Per-M and per-shape breakdown, each timed over its own graph.
    by_m = {}
    for m in DECODE_MS:
        t = time_region(graph_of([c for c in calls if c[0] == m]).replay, steps, 1) / steps
        b = LAYERS * sum(decode_bytes(m, k, n) for k, n in SHAPES)
        by_m[str(m)] = round(b / t / 1e9, 1)
    by_shape = {}
    for si, (k, n) in enumerate(SHAPES):
        for m in DECODE_MS:
            sub = [c for c in calls if c[:3] == (m, k, n)]
            t = time_region(graph_of(sub).replay, steps, 1) / (steps * len(sub))
            by_shape[f"{SHAPE_NAMES[si]}_M{m}"] = {
                "us": round(t * 1e6, 2), "gbps": round(decode_bytes(m, k, n) / t / 1e9, 1)}
    # The drop-in's own k_proj / v_proj (model_runner.py:322-324 calls q, k and v separately):
    # (K, N) = (4096, 1024), over as many rotated copies as keep the same bytes beyond the cache.
    k, n = KV_SHAPE
    kv_weights = make_weights(pkg, dev, k, n, 4 * LAYERS, gen)
    for m in DECODE_MS:
        y_kv = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
        sub = [(m, k, n, (xs[(m, k)].data_ptr(), k, q.data_ptr(), s.data_ptr(), y_kv.data_ptr(),
                          n, m, n, k, 1, ws.data_ptr(), ws_bytes)) for q, s in kv_weights]
        t = time_region(graph_of(sub).replay, steps, 1) / (steps * len(sub))
        by_shape[f"kv_proj_M{m}"] = {
            "us": round(t * 1e6, 2), "gbps": round(decode_bytes(m, k, n) / t / 1e9, 1)}
    # The attention projections as the drop-in runs them: q_proj (the o_proj shape) + k_proj +
    # v_proj as three launches, against the grouped q/k/v (QKVGroup: one stacked qkv launch).
    qkv_drop_in = {}
    for m in DECODE_MS:
        sep = by_shape[f"o_proj_M{m}"]["us"] + 2 * by_shape[f"kv_proj_M{m}"]["us"]
        qkv_drop_in[str(m)] = {"separate_us": round(sep, 2),
                               "grouped_us": by_shape[f"qkv_M{m}"]["us"]}
    return {
        "seconds_per_step": per_step,
        "bytes_per_step": total_bytes,
        "launches_per_step": len(calls),
        "gbps": total_bytes / per_step / 1e9,
        "by_m_gbps": by_m,
        "by_shape": by_shape,
        "qkv_drop_in": qkv_drop_in,
    }


def bench_decode_reference(dev, steps: int, gen, int8_seconds: float) -> dict:
    """The reference engine's own GPU path for the same sweep, as context: every projection a
    bf16 `F.linear` on bf16 weights (model_runner.py:49, 184-200), same shapes, M, rotated
    copies and graph replay. Returns its us per step and the int8 path's speedup over it."""
    import torch

    w16 = [[(torch.randn(n, k, generator=gen) * 0.02).to(torch.bfloat16).to(dev)
            for _ in range(LAYERS)] for k, n in SHAPES]
    xs = {(m, k): torch.randn(m, k, generator=gen).to(torch.bfloat16).to(dev)
          for m in DECODE_MS for k in {k for k, _ in SHAPES}}

    def step():
        for m in DECODE_MS:
            for layer in range(LAYERS):
                for si, (k, _) in enumerate(SHAPES):
                    torch.nn.functional.linear(xs[(m, k)], w16[si][layer])

    t = time_graph(step, steps)
    del w16
    return {"bf16_us_per_step": round(t * 1e6, 1),
            "int8_us_per_step": round(int8_seconds * 1e6, 1),
            "speedup": round(t / int8_seconds, 3)}


def bench_prefill(pkg, dev, steps: int, gen) -> dict:
    """Config 2: the four Llama-3-8B projections (one "layer") at M in PREFILL_MS through the
    tiled kernel, over LAYERS rotated weight copies, replayed from one captured graph as the
    engine's piecewise prefill graphs run them. TFLOP/s of 2MNK and ms per layer."""
    import torch

    weights = [make_weights(pkg, dev, k, n, LAYERS, gen) for k, n in SHAPES]
    res = {}
    for m in PREFILL_MS:
        flops = 0
        xs = []
        for k, n in SHAPES:
            xs.append(torch.randn(m, k, generator=gen).to(torch.bfloat16).to(dev))
            flops += 2 * m * n * k

        def step(xs=xs):
            for layer in range(LAYERS):
                for x, copies in zip(xs, weights):
                    q, s = copies[layer]
                    pkg.ops.w8a16_linear(x, q, s, algo=2)

        t = time_graph(step, 2) / LAYERS
        res[str(m)] = {"tflops": round(flops / t / 1e12, 1), "ms": round(t * 1e3, 3)}
    res["mfma_frac_M2048"] = round(res["2048"]["tflops"] / BF16_PEAK_TFLOPS, 4)
    del weights
    # Context, not the product: the vendor BLAS's bf16 GEMM (F.linear on bf16 weights, no
    # dequantization) on the same shapes, rotated copies and graph replay.
    w16 = [[(torch.randn(n, k, generator=gen) * 0.02).to(torch.bfloat16).to(dev)
            for _ in range(LAYERS)] for k, n in SHAPES]
    for m in PREFILL_MS:
        xs = [torch.randn(m, k, generator=gen).to(torch.bfloat16).to(dev) for k, _ in SHAPES]
        flops = sum(2 * m * n * k for k, n in SHAPES)

        def vstep(xs=xs):
            for layer in range(LAYERS):
                for x, copies in zip(xs, w16):
                    torch.nn.functional.linear(x, copies[layer])

        t = time_graph(vstep, 2) / LAYERS
        res[str(m)]["vendor_bf16_tflops"] = round(flops / t / 1e12, 1)
    del w16
    return res


def bench_w8a8(pkg, dev, steps: int, gen) -> dict:
    """Config 3: per-token quantization then the int8 GEMM, over the four Llama-3-8B shapes (one
    "layer"), at M in W8A8_MS. LAYERS weight copies are rotated (8 x 218 MB, beyond the 256 MB
    Infinity Cache) and the calls replayed from one captured graph, so the HBM-bound small-M
    figures are GPU time, not host launch time. Reports TOP/s (2MNK), ms per layer and GB/s of
    algorithmic bytes (quantizer 3MK + 4M, GEMM K·N + 4N + MK + 4M + 2MN), and from M = 512
    `gemm_tops`: the int8 GEMM with its epilogue alone on x quantized beforehand, the work the
    vendor GEMM figure times."""
    import torch

    weights = [make_weights(pkg, dev, k, n, LAYERS, gen) for k, n in SHAPES]
    res = {}
    for m in W8A8_MS:
        ops = nbytes = 0
        xs = []
        for k, n in SHAPES:
            x = torch.randn(m, k, generator=gen).to(torch.bfloat16)
            x[:, torch.randperm(k, generator=gen)[: round(0.001 * k)]] *= 20
            xs.append(x.to(dev))
            ops += 2 * m * n * k
            nbytes += 3 * m * k + 4 * m + k * n + 4 * n + m * k + 4 * m + 2 * m * n

        def step(xs=xs):
            for layer in range(LAYERS):
                for x, copies in zip(xs, weights):
                    q, s = copies[layer]
                    pkg.ops.w8a8_linear(x, q, s)

        t = time_graph(step, max(2, steps // 4)) / LAYERS
        res[str(m)] = {"tops": round(ops / t / 1e12, 2), "ms": round(t * 1e3, 4),
                       "gbps": round(nbytes / t / 1e9, 1)}
        if m >= 512:
            # The int8 GEMM and its epilogue alone (x quantized beforehand), the same work as
            # the vendor GEMM timed below, plus the bf16 epilogue.
            xqs = [pkg.ops.quantize_act_per_token(x) for x in xs]

            def gemm_step(xqs=xqs):
                for layer in range(LAYERS):
                    for (xq, sx), copies in zip(xqs, weights):
                        q, s = copies[layer]
                        pkg.ops.w8a8_gemm(xq, sx, q, s)

            tg = time_graph(gemm_step, max(2, steps // 4)) / LAYERS
            res[str(m)]["gemm_tops"] = round(ops / tg / 1e12, 1)
            del xqs
    del weights
    # Context, not the product: the vendor BLAS's int8 GEMM (torch._int_mm, int32 out, no
    # quantizer or epilogue) on the same shapes at the prefill-sized M, rotated copies.
    qv = [[torch.randint(-127, 128, (n, k), generator=gen, dtype=torch.int8).to(dev)
           for _ in range(LAYERS)] for k, n in SHAPES]
    for m in (mm for mm in W8A8_MS if mm >= 512):
        xs = [torch.randint(-127, 128, (m, k), generator=gen, dtype=torch.int8).to(dev)
              for k, _ in SHAPES]
        ops = sum(2 * m * n * k for k, n in SHAPES)

        def vstep(xs=xs):
            for layer in range(LAYERS):
                for x, copies in zip(xs, qv):
                    torch._int_mm(x, copies[layer].t())

        try:
            t = time_graph(vstep, 2) / LAYERS
            res[str(m)]["vendor_int_mm_tops"] = round(ops / t / 1e12, 1)
        except RuntimeError as e:  # not every build routes _int_mm to a GPU kernel
            res[str(m)]["vendor_int_mm_tops"] = None
            print(f"[w8a8] vendor int8 GEMM unavailable: {e}", file=sys.stderr, flush=True)
    del qv
    res["rmsnorm_quantize"] = bench_rmsnorm_quantize(pkg, dev, steps, gen)
    return res


def bench_rmsnorm_quantize(pkg, dev, steps: int, gen) -> dict:
    """The decoder norm fused with per-token quantization (hidden 4096) against transformers'
    LlamaRMSNorm followed by the separate quantizer, each replayed from a captured graph of 20
    calls: us per call, and GB/s of algorithmic bytes (x in, weight, xq and sx out)."""
    import torch
    from transformers.models.llama.modeling_llama import LlamaRMSNorm

    k = 4096
    norm = LlamaRMSNorm(k, eps=1e-5).to(device=dev, dtype=torch.bfloat16)
    res = {}
    for m in (64, 2048):
        x = torch.randn(m, k, generator=gen).to(torch.bfloat16).to(dev)
        reps = 20  # calls per graph, so one graph launch does not dominate a few-us call

        def fused(x=x):
            for _ in range(reps):
                pkg.ops.rmsnorm_quantize(x, norm.weight, 1e-5)

        def unfused(x=x):
            for _ in range(reps):
                pkg.ops.quantize_act_per_token(norm(x))

        t = time_graph(fused, steps) / reps
        t0 = time_graph(unfused, steps) / reps
        nbytes = 2 * m * k + 2 * k + m * k + 4 * m
        res[str(m)] = {"fused_us": round(t * 1e6, 2), "fused_gbps": round(nbytes / t / 1e9, 1),
                       "unfused_us": round(t0 * 1e6, 2)}
    return res


GLU_K, GLU_I = 4096, 14336  # Llama-3-8B gate/up: two (14336, 4096) weights


def bench_glu(pkg, dev, steps: int, gen) -> dict:
    """Fused gate_up + SiLU-mul at the Llama-3-8B shape: decode (M in DECODE_MS, over LAYERS weight
    copies, graph-replayed) in GB/s of algorithmic bytes (2IK + 8I + 2MK + 2MI), prefill at
    M = 2048 in TFLOP/s (4MIK), each beside the unfused pair it replaces (the stacked W8A16
    GEMM, then torch's SiLU and product on its bf16 halves)."""
    import torch

    k, i = GLU_K, GLU_I
    weights = []
    for _ in range(LAYERS):
        w = (torch.randn(2 * i, k, generator=gen, device="cpu") * 0.02).to(dev)
        q, s = pkg.ops.quantize_weight_per_channel(w)
        weights.append((pkg.ops.pack_glu(q), pkg.ops.pack_weight(q), s))
        del w, q

    def fused(x, qg, s):
        pkg.ops.w8a16_glu(x, qg, s)

    def unfused(x, qp, s):
        gu = pkg.ops.w8a16_linear(x, qp, s)
        torch.nn.functional.silu(gu[:, :i]) * gu[:, i:]

    def graph_time(fn, xs, copies):
        fn_all = lambda: [fn(xs, *c) for c in copies]  # noqa: E731
        fn_all()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn_all()
        return time_region(g.replay, steps, 1) / (steps * len(copies))

    res = {"I": i, "K": k, "decode": {}}
    for m in DECODE_MS:
        x = torch.randn(m, k, generator=gen).to(torch.bfloat16).to(dev)
        t = graph_time(fused, x, [(qg, s) for qg, _, s in weights])
        t0 = graph_time(unfused, x, [(qp, s) for _, qp, s in weights])
        nbytes = 2 * i * k + 8 * i + 2 * m * k + 2 * m * i
        res["decode"][str(m)] = {"us": round(t * 1e6, 2), "gbps": round(nbytes / t / 1e9, 1),
                                 "unfused_us": round(t0 * 1e6, 2)}
    m = 2048
    x = torch.randn(m, k, generator=gen).to(torch.bfloat16).to(dev)
    t = graph_time(fused, x, [(weights[0][0], weights[0][2])])
    t0 = graph_time(unfused, x, [(weights[0][1], weights[0][2])])
    res["prefill_M2048"] = {"us": round(t * 1e6, 1), "tflops": round(4 * m * i * k / t / 1e12, 1),
                            "mfma_frac": round(4 * m * i * k / t / 1e12 / BF16_PEAK_TFLOPS, 4),
                            "unfused_us": round(t0 * 1e6, 1)}
    return res


TP8_SHARDS = [("qkv", 4096, 768), ("o_proj", 512, 4096), ("gate_up", 4096, 3584),
              ("down", 1792, 4096)]  # (name, K, N) of one GPU's share at tensor parallelism 8


def bench_tp8_shards(pkg, dev, steps: int, gen) -> dict:
    """One GPU's share of each Llama-3-8B projection under 8-way tensor parallelism (column-
    parallel qkv and gate_up split N, row-parallel o_proj and down split K; the all-reduce of the
    row-parallel outputs is not timed): W8A16 decode GB/s at M = 1 and 64 and prefill TFLOP/s at
    M = 2048, each over enough rotated weight copies (at least 768 MB) that every launch streams
    its weight from HBM, replayed from graphs."""
    import torch

    res = {}
    for name, k, n in TP8_SHARDS:
        copies = make_weights(pkg, dev, k, n, -(-768_000_000 // (k * n)), gen)
        row = {}
        for m in (1, 64, 2048):
            x = torch.randn(m, k, generator=gen).to(torch.bfloat16).to(dev)

            def step(x=x):
                for q, s in copies:
                    pkg.ops.w8a16_linear(x, q, s)

            t = time_graph(step, steps) / len(copies)
            if m == 2048:
                row["M2048_tflops"] = round(2.0 * m * n * k / t / 1e12, 1)
            else:
                row[f"M{m}_us"] = round(t * 1e6, 2)
                row[f"M{m}_gbps"] = round(decode_bytes(m, k, n) / t / 1e9, 1)
        res[f"{name}_{k}x{n}"] = row
        del copies
    return res


MID_MS = [64, 65, 128, 129, 256]


def bench_mid_range(pkg, dev, steps: int, gen) -> dict:
    """The four Llama-3-8B shapes just above the decode range, where the tiled GEMM splits K for
    the narrow ones (65..256 tokens; 64 is the decode route, for reference): us per call in
    W8A16 and in W8A8 (activation quantizer included), each over enough rotated weight copies
    (at least 768 MB) that every launch streams its weight from HBM, replayed from graphs."""
    import torch

    res = {"w8a16": {}, "w8a8": {}}
    for name, (k, n) in zip(SHAPE_NAMES, SHAPES):
        copies = make_weights(pkg, dev, k, n, -(-768_000_000 // (k * n)), gen)
        for mode in res:
            row = {}
            for m in MID_MS:
                x = torch.randn(m, k, generator=gen).to(torch.bfloat16).to(dev)
                if mode == "w8a16":
                    def step(x=x):
                        for q, s in copies:
                            pkg.ops.w8a16_linear(x, q, s)
                else:
                    def step(x=x):
                        for q, s in copies:
                            pkg.ops.w8a8_linear(x, q, s)
                row[f"M{m}_us"] = round(time_graph(step, steps) / len(copies) * 1e6, 2)
            res[mode][name] = row
        del copies
    return res


def bench_launch_floor(pkg, dev, steps: int, gen) -> dict:
    """The fixed cost of one kernel in a graph, which bounds the small decode shapes: 64
    back-to-back launches replayed from one graph, per launch, for torch's smallest elementwise
    kernel (an in-place add on 16 floats) and for the decode GEMM on a trivial shape (M = 1,
    K = 64, N = 16: one K step, one row tile) and on a 64 KB weight (K = 4096, N = 16: 64 K
    steps over the workgroup's 8 waves)."""
    import torch

    res = {}
    a = torch.zeros(16, device=dev)

    def add():
        for _ in range(64):
            a.add_(1.0)

    res["torch_elementwise_us"] = round(time_graph(add, steps) / 64 * 1e6, 2)
    lib = pkg.library()
    for k, n in ((64, 16), (4096, 16)):
        w = (torch.randn(n, k, generator=gen) * 0.02).to(dev)
        q, s = pkg.ops.quantize_weight_per_channel(w)
        qp = pkg.ops.pack_weight(q)
        x = torch.randn(1, k, generator=gen).to(torch.bfloat16).to(dev)
        y = torch.empty(1, n, dtype=torch.bfloat16, device=dev)

        def gemm(x=x, qp=qp, s=s, y=y, k=k, n=n):
            stream = torch.cuda.current_stream().cuda_stream
            for _ in range(64):
                st = lib.lse_w8a16_gemm_algo(x.data_ptr(), k, qp.data_ptr(), s.data_ptr(),
                                             y.data_ptr(), n, 1, n, k, 1, None, 0, stream)
                if st:
                    raise RuntimeError(f"lse_w8a16_gemm_algo status {st}")

        res[f"decode_gemm_K{k}_N{n}_us"] = round(time_graph(gemm, steps) / 64 * 1e6, 2)
    return res


def device_peaks() -> dict:
    """The roofline peaks used (AMD's published MI355X figures) beside the ones re-derived on this
    box: CUs x max engine clock (rocminfo) x per-CU dense rate (bf16: 4 SIMDs x 1024 flops per
    clock, the 16x16x32 MFMA's 16 K flops per 16 cycles; int8 twice that)."""
    import re
    import subprocess

    import torch

    props = torch.cuda.get_device_properties(0)
    cus = props.multi_processor_count
    mhz = None
    try:
        info = subprocess.run(["rocminfo"], capture_output=True, text=True, timeout=60).stdout
        gpu = info[info.find(getattr(props, "gcnArchName", "gfx950").split(":")[0]):]
        m = re.search(r"Max Clock Freq\. \(MHz\):\s*(\d+)", gpu)
        mhz = int(m.group(1)) if m else None
    except (OSError, subprocess.SubprocessError):
        pass
    out = {"name": props.name, "arch": getattr(props, "gcnArchName", None), "cus": cus,
           "max_engine_clock_mhz": mhz, "published": {"hbm_gbps": HBM_PEAK_GBPS,
                                                       "bf16_tflops": BF16_PEAK_TFLOPS,
                                                       "int8_tops": INT8_PEAK_TOPS}}
    if mhz:
        out["derived"] = {"bf16_tflops": round(cus * mhz * 1e6 * 4096 / 1e12, 1),
                          "int8_tops": round(cus * mhz * 1e6 * 8192 / 1e12, 1)}
    return out


def bench_lm_head(pkg, dev, steps: int, gen) -> dict:
    """The bf16 lm_head of Llama-3 (N = 128256, K = 4096, 1.05 GB) at decode batch sizes and at
    the row counts a prefill step's `emit_owed` passes (one row per sequence): the packed bf16
    path (`lse_bf16_decode_gemm`) against torch's F.linear (the vendor BLAS, the reference's own
    call), us and GB/s (2NK + 2MK + 2MN bytes), over 2 weight copies so every call streams its
    weight from HBM."""
    import torch

    n, k = 128256, 4096
    ws = [(torch.randn(n, k, generator=gen) * 0.02).to(torch.bfloat16).to(dev) for _ in range(2)]
    wps = [pkg.ops.pack_bf16_weight(w) for w in ws]
    res = {}
    for m in LM_HEAD_MS:
        x = torch.randn(m, k, generator=gen).to(torch.bfloat16).to(dev)
        ours = lambda x=x: [pkg.ops.bf16_decode_linear(x, wp, n) for wp in wps]  # noqa: E731
        blas = lambda x=x: [torch.nn.functional.linear(x, w) for w in ws]  # noqa: E731
        t = time_graph(ours, steps) / 2
        t0 = time_graph(blas, steps) / 2
        nbytes = 2 * n * k + 2 * m * k + 2 * m * n
        res[str(m)] = {"us": round(t * 1e6, 1), "gbps": round(nbytes / t / 1e9, 1),
                       "vendor_blas_us": round(t0 * 1e6, 1),
                       "vendor_blas_gbps": round(nbytes / t0 / 1e9, 1)}
    return res


ATTN_CASES = [  # (name, entries, context, pools rotated, table as wide as the pool)
    ("decode_b64_ctx1025", 64, 1025, 4, False),  # config 4's decode step, one layer
    # the same call in the reference's graphed-decode shape (decode_graph.py:97,149): a block
    # table as wide as the whole pool
    ("decode_b64_ctx1025_pool_wide_table", 64, 1025, 4, True),
    ("decode_b8_ctx8192", 8, 8192, 4, False),    # few sequences, long context: the split path
    ("decode_b256_ctx512", 256, 512, 4, False),
]
ATTN_H, ATTN_HKV, ATTN_D, ATTN_BS = 32, 8, 128, 16


def bench_attention(pkg, dev, steps: int, gen) -> dict:
    """Paged decode attention (one query token per sequence, Llama-3-8B heads, block size 16,
    physical blocks shuffled over the pool): us per call and GB/s of algorithmic bytes (K and V
    rows of every visible position, q in, o out, block table), over `pools` distinct pools so
    each call streams its K/V from HBM; beside it torch's scaled_dot_product_attention on the
    same K/V laid out contiguously (bf16, no paging)."""
    import torch

    res = {}
    h, h_kv, d, bs = ATTN_H, ATTN_HKV, ATTN_D, ATTN_BS
    for name, e, ctx, pools, pool_wide in ATTN_CASES:
        nblk = -(-ctx // bs)
        blocks = e * nblk + 1
        perm = torch.randperm(blocks - 1, generator=gen)
        table = perm[: e * nblk].reshape(e, nblk).to(torch.int32)
        if pool_wide:  # columns past each sequence's blocks name the scratch block
            wide = torch.full((e, blocks), blocks - 1, dtype=torch.int32)
            wide[:, :nblk] = table
            table = wide
        table = table.to(dev)
        kv = [(torch.randn(blocks, bs, h_kv, d, generator=gen).to(torch.bfloat16).to(dev),
               torch.randn(blocks, bs, h_kv, d, generator=gen).to(torch.bfloat16).to(dev))
              for _ in range(pools)]
        q = torch.randn(h, e, d, generator=gen).to(torch.bfloat16).to(dev)
        i32 = lambda v: torch.tensor(v, dtype=torch.int32, device=dev)  # noqa: E731
        ctx_t, qo_t = i32([ctx] * e), i32([ctx - 1] * e)
        qs_t, ql_t = i32(list(range(e))), i32([1] * e)

        def step(kv=kv, q=q, table=table, ctx_t=ctx_t, qo_t=qo_t, qs_t=qs_t, ql_t=ql_t):
            for kp, vp in kv:
                pkg.ops.paged_attention_forward(q, kp, vp, table, ctx_t, qo_t, qs_t, ql_t, bs, 1)

        step()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step()
        t = time_region(g.replay, steps, 1) / (steps * pools)
        nbytes = e * ctx * h_kv * d * 2 * 2 + 2 * (h * e * d * 2) + e * nblk * 4
        # torch SDPA on contiguous (E, H_KV, ctx, D) K/V, GQA by expansion to H heads
        kc = torch.randn(e, h_kv, ctx, d, generator=gen).to(torch.bfloat16).to(dev)
        vc = torch.randn(e, h_kv, ctx, d, generator=gen).to(torch.bfloat16).to(dev)
        qc = q.permute(1, 0, 2).reshape(e, h, 1, d).contiguous()

        def sdpa(kc=kc, vc=vc, qc=qc):
            torch.nn.functional.scaled_dot_product_attention(
                qc, kc, vc, enable_gqa=True)

        sdpa()
        torch.cuda.synchronize()
        t0 = time_region(sdpa, steps, 2) / steps
        res[name] = {"entries": e, "context": ctx, "us": round(t * 1e6, 2),
                     "gbps": round(nbytes / t / 1e9, 1), "frac_of_8TBs": round(nbytes / t / 8e12, 4),
                     "torch_sdpa_contiguous_us": round(t0 * 1e6, 2)}
        del kv, kc, vc
        torch.cuda.empty_cache()
    return res


# ---- profile summaries (CPU only: reads rocprofv3 CSV output) ---------------------------------

SWEEP_CALLS = [(m, si) for m in DECODE_MS for _ in range(LAYERS) for si in range(len(SHAPES))]


def _decode_calls(records: list[dict]) -> list[list[dict]]:
    """Dispatch records (in dispatch order) grouped into decode GEMM calls: a skinny_kernel
    dispatch, plus the skinny_reduce dispatch that follows it when K is split, or the 64 x 128
    tiled_gemm_kernel dispatch the decode path uses for gate_up at 33..64 tokens."""
    calls: list[list[dict]] = []
    for r in records:
        name = r["Kernel_Name"]
        if "skinny_kernel" in name or "tiled_gemm_kernel" in name:
            calls.append([r])
        elif "skinny_reduce" in name:
            calls[-1].append(r)
    return calls


def _short(name: str) -> str:
    return name.split("(")[0].replace("void ", "")


def summarize_profiles(trace_dir: str, fetch_dir: str, write_dir: str) -> None:
    import csv
    import statistics

    def read(path):
        with open(path, newline="") as f:
            return list(csv.DictReader(f))

    n = len(SWEEP_CALLS)
    trace = read(Path(trace_dir) / "run_kernel_trace.csv")
    trace.sort(key=lambda r: int(r["Start_Timestamp"]))
    calls = _decode_calls(trace)
    passes = len(calls) // n
    # Pass 0 is the eager run before capture; the sweep graph's replays follow (warmup + steps),
    # then the per-M and per-shape graphs, which are not used here.
    replays = [calls[i * n:(i + 1) * n] for i in range(1, passes)]
    replays = [r for r in replays
               if [_short(c[0]["Kernel_Name"]) for c in r] ==
               [_short(c[0]["Kernel_Name"]) for c in calls[:n]]][:7]
    span = {}
    for i in range(n):
        span[i] = statistics.median(
            (int(r[i][-1]["End_Timestamp"]) - int(r[i][0]["Start_Timestamp"])) / 1e3
            for r in replays)

    def counters(d, counter):
        rows = [r for r in read(Path(d) / "run_counter_collection.csv")
                if r["Counter_Name"] == counter]
        rows.sort(key=lambda r: int(r["Dispatch_Id"]))
        calib = [float(r["Counter_Value"]) for r in rows if "bitwise_not" in r["Kernel_Name"]]
        factor = CALIBRATION_BYTES / (calib[0] * 1024)
        per_call = [sum(float(r["Counter_Value"]) for r in c) * 1024 * factor
                    for c in _decode_calls(rows)[:n]]
        return factor, calib[0], per_call

    ff, fkib, fetch = counters(fetch_dir, "FETCH_SIZE")
    wf, wkib, write = counters(write_dir, "WRITE_SIZE")

    stats = read(Path(trace_dir) / "run_kernel_stats.csv")
    cmds = [
        "rocprofv3 --kernel-trace --stats -d gpurun_out/prof_decode -o run --output-format csv "
        "-- python3 bench.py --only decode --steps 5 --warmup 2",
        "rocprofv3 --pmc FETCH_SIZE -d gpurun_out/pmc_fetch -o run --output-format csv "
        "-- python3 bench.py --only decode --steps 1 --warmup 0",
        "rocprofv3 --pmc WRITE_SIZE -d gpurun_out/pmc_write -o run --output-format csv "
        "-- python3 bench.py --only decode --steps 1 --warmup 0",
        "python3 bench.py --summarize-profiles gpurun_out/prof_decode gpurun_out/pmc_fetch "
        "gpurun_out/pmc_write",
    ]
    out = ["# skinny_kernel (+ skinny_reduce; tiled_gemm_kernel 64 x 128 for gate_up at 64 "
           "tokens) — config-1 W8A16 decode sweep", "",
           "Llama-3-8B shapes (K, N) in {(4096,6144), (4096,4096), (4096,28672), (14336,4096)} x "
           f"M in {DECODE_MS}, {LAYERS} weight copies rotated, one MI355X.", "",
           "Commands (repository root, one MI355X; the last runs on any host):", "", "```",
           *cmds, "```", "",
           "## rocprofv3 --stats (whole profiled run)", "",
           "| kernel | calls | avg us | total ms |", "|---|---|---|---|"]
    for r in stats:
        if any(t in r["Name"] for t in ("skinny", "tiled_gemm_kernel", "bitwise_not")):
            out.append(f"| `{_short(r['Name'])[:90]}` | {r['Calls']} | "
                       f"{float(r['AverageNs']) / 1e3:.2f} | {float(r['TotalDurationNs']) / 1e6:.2f} |")
    out += ["", f"## Per call (median over {len(replays)} replays of the sweep graph; a call is the "
            "skinny_kernel dispatch plus, when K is split, its skinny_reduce, or one "
            "tiled_gemm_kernel dispatch)", "",
            "HBM bytes = FETCH_SIZE x 1024 x "
            f"{ff:.3f} + WRITE_SIZE x 1024 x {wf:.3f}: the 64 MiB calibration copy read "
            f"{fkib:.1f} KiB of FETCH_SIZE and {wkib:.1f} KiB of WRITE_SIZE.", "",
            "| M | shape (K,N) | kernel | us | algorithmic MB | HBM MB (PMC) | GB/s | frac of 8 TB/s |",
            "|---|---|---|---|---|---|---|---|"]
    tot_t = tot_b = tot_h = 0.0
    seen = set()
    for i, (m, si) in enumerate(SWEEP_CALLS):
        k, nn = SHAPES[si]
        b = decode_bytes(m, k, nn)
        tot_t += span[i]
        tot_b += b
        tot_h += fetch[i] + write[i]
        if (m, si) in seen:
            continue
        seen.add((m, si))
        same = [j for j, c in enumerate(SWEEP_CALLS) if c == (m, si)]
        t = statistics.median(span[j] for j in same)
        h = statistics.median(fetch[j] + write[j] for j in same)
        names = " + ".join(sorted({_short(r["Kernel_Name"]).replace("lse::", "")
                                   for j in same for r in replays[0][j]}))
        out.append(f"| {m} | {SHAPE_NAMES[si]} ({k},{nn}) | `{names}` | {t:.2f} | {b / 1e6:.2f} | "
                   f"{h / 1e6:.2f} | {b / t / 1e3:.0f} | {b / t / 1e3 / HBM_PEAK_GBPS:.3f} |")
    avg_b, avg_h, avg_t = tot_b / n, tot_h / n, tot_t / n
    out += ["", f"Sweep of {n} calls: sum of per-call medians {tot_t:.1f} us; "
            f"{tot_b / 1e9:.3f} GB algorithmic -> {tot_b / tot_t / 1e3:.0f} GB/s "
            f"({tot_b / tot_t / 1e3 / HBM_PEAK_GBPS:.3f} of 8 TB/s). Average per call: "
            f"{avg_b / 1e6:.2f} MB algorithmic, {avg_h / 1e6:.2f} MB HBM traffic "
            f"({avg_h / avg_b:.3f}x), {avg_t:.2f} us."]
    PROFILE_MD.write_text("\n".join(out) + "\n")
    PROFILE_TRAFFIC.write_text(json.dumps({
        "workload": "config1 W8A16 decode sweep",
        "calls": n,
        "algorithmic_bytes_per_call": round(avg_b),
        "hbm_bytes_per_call": round(avg_h),
        "fetch_factor": round(ff, 4),
        "write_factor": round(wf, 4),
        "median_us_per_call": round(avg_t, 3),
        "library_sources_sha16": library_sources_digest(),
    }, indent=1) + "\n")
    print("\n".join(out))


def tiled_calls(trace_dir: str, pmc_dir: str, keep, ms: list[int], k_per_mfma: int,
                passes: int) -> list[tuple]:
    """The tiled GEMM's calls in a kernel trace and a counter run of the same bench command,
    one row per (M, shape): (m, shape name, k, n, kernel names, median us, MFMA instructions,
    MFMA busy cycles, engine clocks), each a median over the calls of the sum over the call's
    dispatches. A call is one dispatch, or two when the GEMM re-tiles the columns of a partial
    last round; consecutive dispatches are grouped into calls by their MFMA instruction counts,
    which sum to the call's (M/16)(N/16)(K/k_per_mfma). A call that splits K is followed by the
    second pass adding the splits (skinny_reduce); its duration is part of the call's. `keep`
    selects the kernel names; every M runs `passes` passes over the four shapes in order."""
    import csv
    import statistics

    def read(path):
        with open(path, newline="") as f:
            return list(csv.DictReader(f))

    every = sorted((r for r in read(Path(trace_dir) / "run_kernel_trace.csv")
                    if keep(r["Kernel_Name"]) or "skinny_reduce" in r["Kernel_Name"]),
                   key=lambda r: int(r["Start_Timestamp"]))
    trace = [r for r in every if keep(r["Kernel_Name"])]
    # reduce[j]: the second-pass dispatches between kept dispatch j and the next kept one.
    reduce: list[list[dict]] = []
    for r in every:
        if keep(r["Kernel_Name"]):
            reduce.append([])
        elif reduce:
            reduce[-1].append(r)
    pmc = collections_by_dispatch([r for r in read(Path(pmc_dir) / "run_counter_collection.csv")
                                   if keep(r["Kernel_Name"])], "tiled_gemm_kernel")
    if len(trace) != len(pmc):
        raise RuntimeError(f"{len(trace)} traced dispatches but {len(pmc)} counted")
    calls: dict = {}
    i = 0
    for m in ms:
        for _ in range(passes):
            for si, (k, n) in enumerate(SHAPES):
                expect = (m // 16) * (n // 16) * (k // k_per_mfma)
                got, idx = 0, []
                while got < expect:
                    got += pmc[i]["SQ_INSTS_MFMA"]
                    idx.append(i)
                    i += 1
                if got != expect:
                    raise RuntimeError(f"dispatches {idx} of M={m} {SHAPE_NAMES[si]}: {got} MFMA "
                                       f"instructions, expected {expect}")
                calls.setdefault((m, si), []).append(idx)
    rows = []
    dur = lambda r: (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3  # noqa: E731
    for m in ms:
        for si, (k, n) in enumerate(SHAPES):
            cs = calls[(m, si)]
            med = lambda f: statistics.median(sum(f(j) for j in c) for c in cs)  # noqa: E731
            short = lambda r: f"`{r['Kernel_Name'].split('(')[0].replace('void lse::', '')}`"  # noqa: E731
            names = " + ".join(short(r) for j in cs[0] for r in [trace[j], *reduce[j]])
            rows.append((m, SHAPE_NAMES[si], k, n, names,
                         med(lambda j: dur(trace[j]) + sum(dur(r) for r in reduce[j])),
                         med(lambda j: pmc[j]["SQ_INSTS_MFMA"]),
                         med(lambda j: pmc[j]["SQ_VALU_MFMA_BUSY_CYCLES"]),
                         med(lambda j: pmc[j]["GRBM_GUI_ACTIVE"]) / XCDS))
    return rows


def summarize_prefill(trace_dir: str, pmc_dir: str) -> None:
    """Per (M, shape) duration, TFLOP/s and MFMA utilisation of the tiled kernel from a kernel
    trace and a counter run of `bench.py --only prefill` (each M runs one eager pass, then three
    graph replays, LAYERS passes each; every pass calls the four shapes in order)."""
    rows = []
    # GRBM_GUI_ACTIVE comes summed over the XCDs: per XCD it is the kernel's length in engine
    # clocks, which gives the clock the kernel actually ran at.
    for m, sn, k, n, name, us, insts, busy, cycles in tiled_calls(
            trace_dir, pmc_dir, lambda name: "tiled_gemm_kernel" in name, PREFILL_MS, 32,
            4 * LAYERS):
        rows.append((m, sn, k, n, name, us, 2.0 * m * n * k / us / 1e6, insts, busy,
                     cycles / us / 1e3, busy / (CUS * SIMDS_PER_CU * cycles)))
    cmds = [
        "rocprofv3 --kernel-trace --stats -d gpurun_out/prof_prefill -o run --output-format csv "
        "-- python3 bench.py --only prefill --steps 8",
        "rocprofv3 --pmc SQ_INSTS_MFMA SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE -d "
        "gpurun_out/pmc_prefill -o run --output-format csv -- python3 bench.py --only prefill "
        "--steps 8",
        "python3 bench.py --summarize-prefill gpurun_out/prof_prefill gpurun_out/pmc_prefill",
    ]
    out = ["# tiled_gemm_kernel — config-2 W8A16 prefill (Llama-3-8B shapes, M in "
           f"{PREFILL_MS}), one MI355X", "",
           "Commands (repository root, one MI355X; the last runs on any host):", "", "```", *cmds,
           "```", "",
           "frac of 2.5 PF: achieved TFLOP/s (2MNK over the kernel-trace duration) over the "
           "dense bf16 peak. Each v_mfma_f32_16x16x32_bf16 keeps a SIMD's matrix core busy 16 "
           "cycles (SQ_INSTS_MFMA x 16 = SQ_VALU_MFMA_BUSY_CYCLES below); 256 CUs x 4 SIMDs at "
           "2.4 GHz is the 2.5 PFLOP/s peak. GRBM_GUI_ACTIVE, reported summed over the 8 XCDs, "
           "gives the kernel's length in engine clocks, hence the clock it ran at; MFMA "
           "utilisation = SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs x those clocks) is the fraction "
           "of matrix-core cycles used at that clock. For kernels under ~100 us the GRBM window "
           "also spans launch overhead (implied clocks above 2.4 GHz), so read those two columns "
           "for the long kernels: under sustained MFMA load the chip holds ~1.8-1.9 GHz, "
           "i.e. ~1.9 PFLOP/s of reachable dense bf16.", "",
           "| M | shape (K,N) | kernel | us | TFLOP/s | frac of 2.5 PF | MFMA instrs | MFMA busy "
           "cycles | clock (GHz) | MFMA utilisation |", "|---|---|---|---|---|---|---|---|---|---|"]
    tot_f = tot_t = 0.0
    for m, sn, k, n, name, us, tf, insts, busy, ghz, util in rows:
        out.append(f"| {m} | {sn} ({k},{n}) | {name} | {us:.1f} | {tf:.0f} | {tf / 2500:.3f} | "
                   f"{insts:,.0f} | {busy:,.0f} | {ghz:.2f} | {util:.3f} |")
        if m == 2048:
            tot_f += 2.0 * m * n * k
            tot_t += us
    out += ["", f"M = 2048, four shapes: {tot_f / 1e9:.0f} GFLOP in {tot_t:.1f} us -> "
            f"{tot_f / tot_t / 1e6:.0f} TFLOP/s ({tot_f / tot_t / 1e6 / 2500:.3f} of 2.5 PFLOP/s)."]
    PROFILE_PREFILL.write_text("\n".join(out) + "\n")
    print("\n".join(out))


def summarize_w8a8(trace_dir: str, pmc_dir: str) -> None:
    """Per (M, shape) duration, TOP/s and int8 MFMA utilisation of the W8A8 tiled GEMM at the
    prefill-sized M of config 3, from a kernel trace and a counter run of `bench.py --only w8a8`
    (each M runs the quantizer + GEMM step, then the GEMM alone on x quantized beforehand
    (`gemm_tops`), each as one eager pass and three graph replays at `--steps 8`, LAYERS passes
    each, every pass the four shapes in order: 8 LAYERS passes of the same GEMM kernels; the
    decode-range M use other kernels and are left out)."""
    def prefill_gemm(name: str) -> bool:  # the int8 tiled GEMM with the default cache policy
        head = name.split("(")[0]
        if "tiled_gemm_kernel<" not in head:
            return False
        # template arguments: I8, BM, BN, WGM, WGN, NST, GLU, NT (streaming loads), BFW, STAGE_Y
        targs = [t.strip() for t in head[head.index("<") + 1:head.rindex(">")].split(",")]
        return targs[0] == "true" and targs[7] == "false"

    ms = [m for m in W8A8_MS if m > 64]
    rows = []
    for m, sn, k, n, name, us, insts, busy, cycles in tiled_calls(
            trace_dir, pmc_dir, prefill_gemm, ms, 64, 8 * LAYERS):
        rows.append((m, sn, k, n, name, us, 2.0 * m * n * k / us / 1e6, insts, busy,
                     cycles / us / 1e3, busy / (CUS * SIMDS_PER_CU * cycles)))
    cmds = [
        "rocprofv3 --kernel-trace --stats -d gpurun_out/prof_w8a8 -o run --output-format csv -- "
        "python3 bench.py --only w8a8 --steps 8",
        "rocprofv3 --pmc SQ_INSTS_MFMA SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE -d "
        "gpurun_out/pmc_w8a8 -o run --output-format csv -- python3 bench.py --only w8a8 --steps 8",
        "python3 bench.py --summarize-w8a8 gpurun_out/prof_w8a8 gpurun_out/pmc_w8a8",
    ]
    out = ["# tiled_gemm_kernel<true, ...> — config-3 W8A8 int8 GEMM at prefill M (Llama-3-8B "
           f"shapes, M in {ms}), one MI355X", "",
           "Commands (repository root, one MI355X; the last runs on any host):", "", "```", *cmds,
           "```", "",
           "frac of 5.0 POP/s: achieved TOP/s (2MNK over the kernel-trace duration of the GEMM "
           "alone, without the per-token quantizer) over the dense int8 peak. Each "
           "v_mfma_i32_16x16x64_i8 keeps a SIMD's matrix core busy 16 cycles (SQ_INSTS_MFMA x 16 = "
           "SQ_VALU_MFMA_BUSY_CYCLES); 256 CUs x 4 SIMDs at 2.4 GHz is the 5.0 POP/s peak. "
           "GRBM_GUI_ACTIVE, summed over the 8 XCDs, gives the kernel's length in engine clocks "
           "and so the clock it ran at; MFMA utilisation = SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs "
           "x those clocks). Kernels under ~100 us include launch overhead in the GRBM window "
           "(implied clocks above 2.4 GHz): read the utilisation of the long ones.", "",
           "| M | shape (K,N) | kernel | us | TOP/s | frac of 5.0 POP/s | MFMA instrs | MFMA busy "
           "cycles | clock (GHz) | MFMA utilisation |", "|---|---|---|---|---|---|---|---|---|---|"]
    for m in ms:
        tot_o = tot_t = 0.0
        for rm, sn, k, n, name, us, tops, insts, busy, ghz, util in rows:
            if rm != m:
                continue
            out.append(f"| {m} | {sn} ({k},{n}) | {name} | {us:.1f} | {tops:.0f} | "
                       f"{tops / INT8_PEAK_TOPS:.3f} | {insts:,.0f} | {busy:,.0f} | {ghz:.2f} | "
                       f"{util:.3f} |")
            tot_o += 2.0 * m * n * k
            tot_t += us
        out.append(f"| {m} | four shapes | | {tot_t:.1f} | {tot_o / tot_t / 1e6:.0f} | "
                   f"{tot_o / tot_t / 1e6 / INT8_PEAK_TOPS:.3f} | | | | |")
    PROFILE_W8A8.write_text("\n".join(out) + "\n")
    print("\n".join(out))


def summarize_glu(trace_dir: str) -> None:
    """Per-kernel durations of `bench.py --only glu` from a kernel trace: the fused kernels (last
    template argument true) and the unfused GEMMs and elementwise kernels they replace, grouped
    by kernel and grid (M = 1 and M = 8 share the M <= 16 kernel and grid)."""
    import csv
    import statistics

    with open(Path(trace_dir) / "run_kernel_trace.csv", newline="") as f:
        trace = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    groups: dict[tuple[str, int], list[float]] = {}
    for r in trace:
        name = r["Kernel_Name"]
        kernels = ("skinny_kernel", "tiled_gemm_kernel", "silu", "BinaryFunctor")
        if not any(t in name for t in kernels):
            continue
        short = name.split("(")[0].replace("void ", "").replace("lse::", "")
        if "at::native" in short:
            short = "torch silu" if "silu" in name else "torch mul"
        key = (short, int(r["Grid_Size_X"]))
        groups.setdefault(key, []).append(
            (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    cmds = [
        "rocprofv3 --kernel-trace --stats -d gpurun_out/prof_glu -o run --output-format csv -- "
        "python3 bench.py --only glu --steps 5",
        "python3 bench.py --summarize-glu gpurun_out/prof_glu",
    ]
    out = [f"# Fused gate_up + SiLU-mul kernels (I = {GLU_I}, K = {GLU_K}), one MI355X", "",
           "Commands (repository root, one MI355X; the last runs on any host):", "", "```", *cmds,
           "```", "",
           "Fused kernels carry `true` as their last template argument; the unfused pair they "
           "replace is the stacked GEMM (same kernel family, `false`) followed by torch's SiLU "
           "and product on its bf16 halves. Decode launches rotate 8 weight copies (940 MB), so "
           "every launch streams its weights from HBM. Durations are kernel-trace "
           "end - start.", "",
           "| kernel | grid | dispatches | median us | min us |", "|---|---|---|---|---|"]
    for (short, grid), ds in sorted(groups.items(), key=lambda kv: (kv[0][0], kv[0][1])):
        out.append(f"| `{short}` | {grid} | {len(ds)} | {statistics.median(ds):.2f} | "
                   f"{min(ds):.2f} |")
    PROFILE_GLU.write_text("\n".join(out) + "\n")
    print("\n".join(out))


LM_HEAD_MS = DECODE_MS + [128, 256]


def summarize_lm_head(trace_dir: str, steps: int = 5) -> None:
    """Per-M kernel durations of `bench.py --only lm-head --steps 5` from a kernel trace: the
    packed bf16 path (lse kernels) against the vendor BLAS's F.linear, in bench order (for each M
    the packed path, then the vendor's; each a graph of 2 calls, run eagerly once, then
    replayed steps + 1 times, so 2 (steps + 2) calls per block; a call may take several vendor
    kernels)."""
    import csv
    import statistics

    with open(Path(trace_dir) / "run_kernel_trace.csv", newline="") as f:
        trace = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    blocks: list[list[dict]] = []
    for r in trace:
        # The GEMM kernels only: not the packing of the two weight copies, buffer copies, or
        # the small fills that graph capture launches.
        name = r["Kernel_Name"]
        if "pack_bf16" in name or not ("lse::" in name or "Cijk" in name):
            continue
        ours = "lse::" in name
        if not blocks or ("lse::" in blocks[-1][0]["Kernel_Name"]) != ours:
            blocks.append([])
        blocks[-1].append(r)
    calls = 2 * (steps + 2)
    if len(blocks) != 2 * len(LM_HEAD_MS):
        raise RuntimeError(f"{len(blocks)} kernel blocks, expected {2 * len(LM_HEAD_MS)}")
    dur = lambda r: (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3  # noqa: E731
    n, k = 128256, 4096
    cmds = [
        "rocprofv3 --kernel-trace --stats -d gpurun_out/prof_head -o run --output-format csv -- "
        "python3 bench.py --only lm-head --steps 5",
        "python3 bench.py --summarize-lm-head gpurun_out/prof_head",
    ]
    out = [f"# Packed bf16 lm_head (N = {n}, K = {k}, 1.05 GB bf16) against the vendor BLAS, "
           "one MI355X", "", "Commands (repository root, one MI355X; the last runs on any host):",
           "", "```", *cmds, "```", "",
           "Two weight copies rotate, so every call streams its 1.05 GB from HBM. A call's time is "
           "the sum of its kernels' trace durations (end - start); medians over the block's "
           f"{calls} calls. GB/s = (2NK + 2MK + 2MN) / time.", "",
           "| M | packed kernel | packed us | packed GB/s | vendor kernels | vendor us | "
           "vendor GB/s |", "|---|---|---|---|---|---|---|"]
    for mi, m in enumerate(LM_HEAD_MS):
        row = [str(m)]
        for b in blocks[2 * mi:2 * mi + 2]:
            per = len(b) // calls
            if per * calls != len(b):
                raise RuntimeError(f"M={m}: {len(b)} dispatches for {calls} calls")
            us = statistics.median(sum(dur(r) for r in b[c * per:(c + 1) * per])
                                   for c in range(calls))
            names = sorted({r["Kernel_Name"].split("(")[0].replace("void ", "")
                            .replace("lse::", "")[:70] for r in b})
            row += [" + ".join(f"`{s}`" for s in names), f"{us:.1f}",
                    f"{(2 * n * k + 2 * m * k + 2 * m * n) / us / 1e3:.0f}"]
        out.append("| " + " | ".join(row) + " |")
    PROFILE_HEAD.write_text("\n".join(out) + "\n")
    print("\n".join(out))


def summarize_decode_step(trace_dir: str, steps: int = 20, layers: int = 32) -> None:
    """Config 4's int8 linear stack by kernel, from a kernel trace of
    `bench.py --only decode-step-linears --steps 20`: the dispatches after the marker kernel are
    (steps + 2) passes of one step (an eager pass, a warm-up replay, the timed replays); the
    last `steps` passes are summarized. Each dispatch is attributed to its projection by its
    place in the layer's sequence (q/k/v, o_proj, gate/up, down_proj and, when down_proj splits
    K, its second pass)."""
    import csv

    with open(Path(trace_dir) / "run_kernel_trace.csv", newline="") as f:
        trace = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    marks = [i for i, r in enumerate(trace) if DECODE_STEP_MARKER in r["Kernel_Name"]]
    if not marks:
        raise RuntimeError(f"no {DECODE_STEP_MARKER} marker in the trace")
    after = [r for r in trace[marks[-1] + 1:] if "lse::" in r["Kernel_Name"]]
    if len(after) % (steps + 2):
        raise RuntimeError(f"{len(after)} dispatches after the marker for {steps + 2} passes")
    per = len(after) // (steps + 2)
    if per % layers:
        raise RuntimeError(f"{per} dispatches per step for {layers} layers")
    per_layer = per // layers
    names = ["qkv (4096 -> 6144)", "o_proj (4096 -> 4096)", "gate_up + SiLU-mul (4096 -> 2 x 14336)",
             "down (14336 -> 4096)", "down, second pass"][:per_layer]
    timed = after[-steps * per:]
    dur = lambda r: (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3  # noqa: E731
    span = [(int(timed[k * per + per - 1]["End_Timestamp"])
             - int(timed[k * per]["Start_Timestamp"])) / 1e3 for k in range(steps)]
    rows: dict[tuple[str, str], list[float]] = {}
    for k in range(steps):
        for i in range(per):
            r = timed[k * per + i]
            key = (names[i % per_layer], _short(r["Kernel_Name"]).replace("lse::", ""))
            rows.setdefault(key, []).append(dur(r))
    total = sum(sum(v) for v in rows.values()) / steps
    m, hid, inter = 64, 4096, 14336
    wbytes = {names[0]: 4096 * 6144, names[1]: 4096 * 4096, names[2]: 4096 * 2 * inter,
              names[3]: inter * 4096}
    cmds = ["rocprofv3 --kernel-trace --stats -d gpurun_out/prof_step -o run --output-format csv "
            "-- python3 bench.py --only decode-step-linears --steps 20",
            "python3 bench.py --summarize-decode-step gpurun_out/prof_step"]
    out = ["# Config 4: the int8 (W8A16) linear stack of one Llama-3-8B decode step, by kernel, "
           "one MI355X", "", "Commands (repository root, one MI355X; the last runs on any host):",
           "", "```", *cmds, "```", "",
           f"32 layers at M = {m} tokens, captured in one graph; {steps} replays summarized (after "
           "an eager pass and a warm-up replay). A kernel's time is its trace duration "
           "(end - start); per step = the sum over its dispatches in one replay, averaged over "
           "the replays. GB/s = the projection's algorithmic bytes (int8 weights, fp32 scales, "
           "bf16 activations in and out) per layer / its kernels' time per layer.", "",
           "| projection | kernel | calls per step | us per call | us per step | share | GB/s |",
           "|---|---|---|---|---|---|---|"]
    for (proj, kern), ds in rows.items():
        calls = len(ds) // steps
        us_step = sum(ds) / steps
        gb = ""
        if proj in wbytes:
            w = wbytes[proj]
            n = w // (inter if proj == names[3] else hid)
            k_in = inter if proj == names[3] else hid
            n_out = inter if proj == names[2] else n
            nbytes = w + 4 * n + 2 * m * k_in + 2 * m * n_out
            layer_us = sum(v for (pp, _), vs in rows.items() if pp == proj for v in vs) / (steps * layers)
            if proj == names[3] and len(names) > 4:
                layer_us += sum(v for (pp, _), vs in rows.items() if pp == names[4]
                                for v in vs) / (steps * layers)
            gb = f"{nbytes / layer_us / 1e3:.0f}"
        out.append(f"| {proj} | `{kern}` | {calls} | {us_step / calls:.2f} | {us_step:.1f} | "
                   f"{us_step / total:.3f} | {gb} |")
    import statistics
    out += ["", f"Sum of kernel durations per step: {total:.1f} us; first-to-last dispatch span "
            f"per replay: median {statistics.median(span):.1f} us (the difference is the gap "
            "between consecutive kernels in the graph)."]
    PROFILE_STEP.write_text("\n".join(out) + "\n")
    print("\n".join(out))


def summarize_attention(trace_dir: str) -> None:
    """Kernel-trace durations of `bench.py --only attention`: the paged_attn_kernel dispatches,
    in order, fall into one equal run per ATTN_CASES entry (each case dispatches the same
    count); paged_attn_merge runs only for split cases and is matched to them by time."""
    import csv
    import statistics

    with open(Path(trace_dir) / "run_kernel_trace.csv", newline="") as f:
        trace = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    main = [r for r in trace if "paged_attn_kernel" in r["Kernel_Name"]]
    merge = [r for r in trace if "paged_attn_merge" in r["Kernel_Name"]]
    per = len(main) // len(ATTN_CASES)
    dur = lambda r: (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3  # noqa: E731
    h, h_kv, d, bs = ATTN_H, ATTN_HKV, ATTN_D, ATTN_BS
    cmds = [
        "rocprofv3 --kernel-trace --stats -d gpurun_out/prof_att -o run --output-format csv -- "
        "python3 bench.py --only attention --steps 5",
        "python3 bench.py --summarize-attention gpurun_out/prof_att",
    ]
    out = ["# paged_attn_kernel — decode attention over a paged K/V pool, one MI355X", "",
           "Commands (repository root, one MI355X; the last runs on any host):", "", "```", *cmds,
           "```", "",
           f"Llama-3-8B heads (H = {h}, H_KV = {h_kv}, D = {d}), block size {bs}, one query token "
           "per sequence, physical blocks shuffled over the pool, 4 pools rotated so each call "
           "streams its K/V from HBM. Algorithmic bytes = K and V rows of every visible position "
           "+ q + o + block table. Durations are kernel-trace end - start (median); a split case "
           "adds its paged_attn_merge pass.", "",
           "| case | sequences | context | grid | kernel us | merge us | algorithmic MB | GB/s | "
           "frac of 8 TB/s |", "|---|---|---|---|---|---|---|---|---|"]
    for ci, (name, e, ctx, _pools, _wide) in enumerate(ATTN_CASES):
        block = main[ci * per:(ci + 1) * per]
        t0, t1 = int(block[0]["Start_Timestamp"]), int(block[-1]["End_Timestamp"])
        ms = [dur(r) for r in merge if t0 <= int(r["Start_Timestamp"]) <= t1 + 1_000_000]
        us = statistics.median(dur(r) for r in block)
        mus = statistics.median(ms) if ms else 0.0
        nblk = -(-ctx // bs)
        nbytes = e * ctx * h_kv * d * 4 + 4 * h * e * d + 4 * e * nblk
        gbps = nbytes / ((us + mus) * 1e3)
        out.append(f"| {name} | {e} | {ctx} | {block[0]['Grid_Size_X']} | {us:.2f} | "
                   f"{mus:.2f} | {nbytes / 1e6:.1f} | {gbps:.0f} | {gbps / 8000:.3f} |")
    PROFILE_ATTN.write_text("\n".join(out) + "\n")
    print("\n".join(out))


def collections_by_dispatch(rows: list[dict], kernel: str) -> list[dict]:
    """Counter rows of one --pmc run -> one {counter: value} dict per dispatch of `kernel`, in
    dispatch order."""
    by: dict[int, dict] = {}
    for r in rows:
        if kernel in r["Kernel_Name"]:
            by.setdefault(int(r["Dispatch_Id"]), {})[r["Counter_Name"]] = float(r["Counter_Value"])
    return [by[d] for d in sorted(by)]


def library_sources_digest() -> str:
    """First 16 hex digits of the SHA-256 over the HIP sources (file names and contents, sorted):
    a PMC traffic figure is only reported for the library build it was measured on."""
    h = hashlib.sha256()
    for f in sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.h")):
        h.update(f.name.encode())
        h.update(f.read_bytes())
    return h.hexdigest()[:16]


def measured_traffic(dec: dict) -> tuple[float | None, str]:
    """(HBM bytes per decode launch from the committed PMC summary of this same sweep, or None;
    why None). The summary counts only if it covers the same launches and was measured on a
    library built from the current sources."""
    try:
        t = json.loads(PROFILE_TRAFFIC.read_text())
    except (OSError, ValueError):
        return None, f"no readable {PROFILE_TRAFFIC.name}"
    if t.get("calls") != dec["launches_per_step"]:
        return None, "the PMC summary covers another set of launches"
    if t.get("library_sources_sha16") != library_sources_digest():
        return None, "the PMC summary was measured on another build of the kernels"
    return t["hbm_bytes_per_call"], ""


def bench_eager_overhead(pkg, dev, steps: int, gen, calls: int = 500) -> dict:
    """Host cost of eager `Int8Linear` calls (Python validation, the workspace query and
    torch.empty, the ctypes launch), which an eager caller pays per projection (the reference's
    forward_fused, model_runner.py:202-211, and the attention between piecewise segments): the
    o_proj shape at M = 1, `calls` calls back to back. host_submit_us = host time per call
    before the final synchronisation; eager_us = wall time per call including it; beside them
    the device time per call (50 calls replayed from one graph, so the graph launch itself is
    spread over them), and torch's eager bf16 F.linear on the same shape."""
    import time

    import torch

    from llm_serving_engine_amd.int8_linear import Int8Linear

    k, n = 4096, 4096
    lin = torch.nn.Linear(k, n, bias=False, device=dev, dtype=torch.bfloat16)
    mod = Int8Linear.from_linear(lin)
    x = torch.randn(1, k, generator=gen).to(torch.bfloat16).to(dev)

    def loop(fn):
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(calls):
            fn()
        t1 = time.perf_counter()
        torch.cuda.synchronize()
        return (t1 - t0) / calls, (time.perf_counter() - t0) / calls

    submit, eager = loop(lambda: mod(x))
    f_submit, f_eager = loop(lambda: torch.nn.functional.linear(x, lin.weight))
    graph = time_graph(lambda: [mod(x) for _ in range(50)], steps) / 50
    return {"shape": "o_proj (4096, 4096), M = 1", "calls": calls,
            "host_submit_us": round(submit * 1e6, 2), "eager_us": round(eager * 1e6, 2),
            "graph_replay_us_per_call": round(graph * 1e6, 2),
            "bf16_F_linear_host_submit_us": round(f_submit * 1e6, 2),
            "bf16_F_linear_eager_us": round(f_eager * 1e6, 2)}


def time_graph(fn, steps: int) -> float:
    """Seconds per replay of fn captured into one graph."""
    import torch

    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return time_region(g.replay, steps, 1) / steps


DECODE_STEP_MARKER = "quantize_act_rows"  # the kernel launched once before the timed replays


def bench_decode_step_linears(pkg, dev, steps: int, layers: int = 32, batch: int = 64) -> dict:
    """Config 4's int8 (W8A16) linear stack alone, for a kernel trace: a random-init
    Llama-3-8B-architecture model quantized as the decode-step runner quantizes it (fused q/k/v,
    o_proj, fused gate/up with its SiLU-mul, down_proj), the 32 layers' projections at M = batch
    captured in one graph; one eager pass, one warm-up replay, then `steps` replays. A W8A8
    activation quantization of one row is launched just before, as a marker the trace summary
    (`--summarize-decode-step`) starts from."""
    import torch

    from llm_serving_engine_amd.decode_step import DecodeRunner, random_llama

    model = random_llama(layers, seed=4000, device=dev)
    runner = DecodeRunner(model, batch, 8)
    runner.quantize("int8")
    runner.use("int8")
    calls = runner.linear_calls(batch)
    nbytes = runner.linear_bytes(batch)
    marker = torch.zeros(1, 16, dtype=torch.bfloat16, device=dev)
    pkg.ops.quantize_act_per_token(marker)
    t = time_graph(lambda: [mod(x) for mod, x in calls], steps)
    return {"layers": layers, "batch": batch, "replays": steps,
            "int8_linear_us_per_step": round(t * 1e6, 1),
            "int8_linear_gbps": round(nbytes / t / 1e9, 1), "int8_linear_bytes": nbytes}


def bench_decode_step(pkg, dev, steps: int, layers: int = 32, batch: int = 64,
                      context: int = 1024, decode_steps: int = 4) -> dict:
    """Config 4: a random-init Llama-3-8B-architecture model (lm_head bf16), `batch` sequences
    prefilled to `context` tokens by the bf16 model, then `decode_steps` teacher-forced decode
    steps with bf16 linears (the reference path) and with int8 W8A16 linears, from the same KV
    state. Reports the per-step linear time of each stack (replayed from a captured graph at
    M = batch; both include the MLP's SiLU-mul, a separate call on bf16 and inside the fused
    gate/up kernel on int8), aggregate HBM GB/s, the greedy next-token match rate against the
    bf16 reference (limited by quantization: random-init logits are nearly flat) and against an
    eager torch restatement of the same int8 weights (the kernels' own parity), and the top-2
    logit margin."""
    import torch

    from llm_serving_engine_amd.decode_step import DecodeRunner, random_llama

    def note(msg: str) -> None:
        print(f"[decode-step] {msg}", file=sys.stderr, flush=True)

    model = random_llama(layers, seed=4000, device=dev)
    note(f"model ready: {layers} layers")
    runner = DecodeRunner(model, batch, context + decode_steps)
    gen = torch.Generator().manual_seed(4001)
    vocab = model.config.vocab_size
    prompt = torch.randint(0, vocab, (batch, context), generator=gen).to(dev)
    runner.prefill(prompt)
    torch.cuda.synchronize()
    note(f"prefilled {batch} x {context}")
    tok = torch.randint(0, vocab, (batch,), generator=gen).to(dev)
    inputs, ref_top, margins = [], [], []
    for t in range(decode_steps):
        inputs.append(tok)
        logits = runner.step(tok, context + t).float()
        top2 = logits.topk(2, dim=-1)
        ref_top.append(top2.indices[:, 0])
        margins.append((top2.values[:, 0] - top2.values[:, 1]) / logits.std(dim=-1))
        tok = top2.indices[:, 0]
    bf16_calls = runner.linear_calls(batch)
    bf16_bytes = runner.linear_bytes(batch)
    t_bf16 = time_graph(lambda: [mod(x) for mod, x in bf16_calls], steps)
    note("bf16 steps and linear stack timed")
    runner.quantize("int8")
    runner.use("int8")
    note("quantized")
    match = match_torch = 0
    rel = []
    for t in range(decode_steps):
        runner.use("int8-torch")
        restated = runner.step(inputs[t], context + t).float()
        runner.use("int8")
        logits = runner.step(inputs[t], context + t).float()
        rel.append(float((logits - restated).norm() / restated.norm()))
        top = logits.argmax(-1)
        match += int((top == ref_top[t]).sum())
        match_torch += int((top == restated.argmax(-1)).sum())
    # Layer-wise error: each projection of one step against the fp64 product of the input the
    # kernel saw (gate_up: fp64 silu(g) * u), as max|y - golden| / max|golden|.
    runner.trace = []
    runner.step(inputs[-1], context + decode_steps - 1)
    worst = 0.0
    for i, name, x, y in runner.trace:
        mod = runner.int8[i][name]
        q, s = mod.unpacked_qweight().double(), mod.scales.double()
        xd = x.reshape(-1, x.shape[-1]).double()
        if name == "gate_up":
            inter = mod.intermediate_size
            g = (xd @ q[:inter].t()) * s[:inter]
            golden = torch.nn.functional.silu(g) * ((xd @ q[inter:].t()) * s[inter:])
        else:
            golden = (xd @ q.t()) * s
        err = (y.reshape(golden.shape).double() - golden).abs().max() / golden.abs().max()
        worst = max(worst, float(err))
    traced = len(runner.trace)
    runner.trace = None
    int8_calls = runner.linear_calls(batch)
    int8_bytes = runner.linear_bytes(batch)
    t_int8 = time_graph(lambda: [mod(x) for mod, x in int8_calls], steps)
    # Whole decode steps (embedding to logits), each captured in a graph at the last position:
    # int8 and bf16 linears, each with the HIP paged attention and with the fp32 torch attention
    # over the contiguous cache.
    runner.enable_paged()
    pos = context + decode_steps - 1
    tok = inputs[-1]
    runner.use_attention("paged")
    paged_logits = runner.step(tok, pos).float()
    t_step_paged = time_graph(lambda: runner.step(tok, pos), steps)
    runner.use_attention("torch")
    torch_logits = runner.step(tok, pos).float()
    t_step_int8 = time_graph(lambda: runner.step(tok, pos), steps)
    runner.use("bf16")
    t_step_bf16 = time_graph(lambda: runner.step(tok, pos), steps)
    runner.use_attention("paged")
    t_step_bf16_paged = time_graph(lambda: runner.step(tok, pos), steps)
    runner.use_attention("torch")
    note("whole steps timed")
    h = torch.randn(batch, model.config.hidden_size, generator=gen).to(torch.bfloat16).to(dev)
    t_head = time_graph(lambda: model.lm_head(h), steps)
    t_head_packed = time_graph(lambda: runner.head(h), steps)
    head_bytes = 2 * model.lm_head.weight.numel()
    margin = torch.cat(margins)
    return {
        "layers": layers, "batch": batch, "context": context,
        "int8_linear_us_per_step": round(t_int8 * 1e6, 1),
        "int8_linear_gbps": round(int8_bytes / t_int8 / 1e9, 1),
        "int8_linear_bytes": int8_bytes,
        "bf16_linear_us_per_step": round(t_bf16 * 1e6, 1),
        "bf16_linear_gbps": round(bf16_bytes / t_bf16 / 1e9, 1),
        "step_us_int8_paged_attention": round(t_step_paged * 1e6, 1),
        "step_us_int8_torch_attention": round(t_step_int8 * 1e6, 1),
        "step_us_bf16_torch_attention": round(t_step_bf16 * 1e6, 1),
        "step_us_bf16_paged_attention": round(t_step_bf16_paged * 1e6, 1),
        "paged_vs_torch_attention_logit_rel_diff": round(
            float((paged_logits - torch_logits).norm() / torch_logits.norm()), 5),
        "lm_head_bf16_us": round(t_head * 1e6, 1),
        "lm_head_gbps": round(head_bytes / t_head / 1e9, 1),
        "lm_head_packed_us": round(t_head_packed * 1e6, 1),
        "lm_head_packed_gbps": round(head_bytes / t_head_packed / 1e9, 1),
        "greedy_match_rate": round(match / (batch * decode_steps), 4),
        "greedy_match_rate_vs_int8_torch_restatement": round(
            match_torch / (batch * decode_steps), 4),
        "logit_rel_diff_vs_int8_torch_restatement": round(max(rel), 5),
        "layerwise_projections_checked": traced,
        "layerwise_worst_max_abs_over_max_golden": round(worst, 6),
        "tokens_compared": batch * decode_steps,
        "top2_margin_over_logit_std": {"median": round(float(margin.median()), 4),
                                       "min": round(float(margin.min()), 5)},
    }


def main() -> None:
    args = parse()
    if args.summarize_profiles:
        summarize_profiles(*args.summarize_profiles)
        return
    if args.summarize_prefill:
        summarize_prefill(*args.summarize_prefill)
        return
    if args.summarize_decode_step:
        summarize_decode_step(args.summarize_decode_step)
        return
    if args.summarize_w8a8:
        summarize_w8a8(*args.summarize_w8a8)
        return
    if args.summarize_glu:
        summarize_glu(args.summarize_glu)
        return
    if args.summarize_lm_head:
        summarize_lm_head(args.summarize_lm_head)
        return
    if args.summarize_attention:
        summarize_attention(args.summarize_attention)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the int8 Linear "
              "path runs on a single MI355X; multi-GPU sharding is a design note only)",
              file=sys.stderr)
        sys.exit(2)
    import torch

    import __graft_entry__

    pkg = __graft_entry__.load_package()
    dev = torch.device("cuda:0")
    gen = torch.Generator().manual_seed(1000)
    out: dict = {}

    if args.only == "decode":
        calibration_copy(dev)
    if args.only in (None, "decode"):
        dec = bench_decode(pkg, dev, args.steps, args.warmup, gen)
    if args.only == "prefill":
        print(json.dumps({"prefill": bench_prefill(pkg, dev, args.steps, gen)}))
        return
    if args.only == "w8a8":
        print(json.dumps({"w8a8": bench_w8a8(pkg, dev, args.steps, gen)}))
        return
    if args.only == "glu":
        print(json.dumps({"fused_gate_up": bench_glu(pkg, dev, args.steps, gen)}))
        return
    if args.only == "lm-head":
        print(json.dumps({"lm_head_bf16": bench_lm_head(pkg, dev, args.steps, gen)}))
        return
    if args.only == "attention":
        print(json.dumps({"paged_attention": bench_attention(pkg, dev, args.steps, gen)}))
        return
    if args.only == "decode-step":
        print(json.dumps({"decode_step": bench_decode_step(pkg, dev, args.steps)}))
        return
    if args.only == "decode-step-linears":
        print(json.dumps({"decode_step_linears": bench_decode_step_linears(pkg, dev,
                                                                           args.steps)}))
        return
    if args.only == "mid":
        print(json.dumps({"mid_range": bench_mid_range(pkg, dev, args.steps, gen)}))
        return
    if args.only == "tp8":
        print(json.dumps({"tp8_shard_shapes": bench_tp8_shards(pkg, dev, args.steps, gen),
                          "device": device_peaks()}))
        return

    secondary = {}
    if not args.no_secondary and args.only is None:
        secondary["prefill_w8a16"] = bench_prefill(pkg, dev, args.steps, gen)
        secondary["w8a8"] = bench_w8a8(pkg, dev, args.steps, gen)
        secondary["fused_gate_up"] = bench_glu(pkg, dev, args.steps, gen)
        secondary["paged_attention"] = bench_attention(pkg, dev, args.steps, gen)
        secondary["decode_vs_reference_bf16"] = bench_decode_reference(
            dev, args.steps, gen, dec["seconds_per_step"])
        secondary["eager_int8_linear"] = bench_eager_overhead(pkg, dev, args.steps, gen)
        secondary["tp8_shard_shapes"] = bench_tp8_shards(pkg, dev, args.steps, gen)
        secondary["mid_range"] = bench_mid_range(pkg, dev, args.steps, gen)
        secondary["launch_floor"] = bench_launch_floor(pkg, dev, args.steps, gen)
        torch.cuda.empty_cache()
        secondary["decode_step"] = bench_decode_step(pkg, dev, args.steps)
        secondary["device"] = device_peaks()

    cpu = cpu_int8 = None
    if not args.no_cpu and args.only is None:
        from oracle.cpu_baseline import time_bf16_linear_sweep, time_int8_restatements

        c = time_bf16_linear_sweep(SHAPES, DECODE_MS, budget_s=20.0)
        cpu = {
            "value": round(c["gbps"], 2),
            "unit": "GB/s",
            "cores": c["threads"],
            "kind": "port",
            "sample": ("reference path bf16 F.linear on the host CPU "
                       f"({c['cpu']}), one layer of each config-1 shape at M in {DECODE_MS}, "
                       "median of 5"),
        }
        r = time_int8_restatements(SHAPES, DECODE_MS, budget_s=10.0)
        cpu_int8 = {
            "unit": "GB/s",
            "cores": r["threads"],
            "w8a16_weight_int8pack_mm": round(r["w8a16_weight_int8pack_mm"]["gbps"], 2),
            "w8a8_quantize_int_mm": round(r["w8a8_int_mm"]["gbps"], 2),
            "sample": ("torch's int8 CPU kernels for the same layers and M, same bytes unit, "
                       "median of 5"),
        }

    gbps = dec["gbps"]
    traffic, why = measured_traffic(dec)
    out = {
        "metric": "HBM GB/s at decode M<=64 + TOPS at prefill M=2048, Llama-3-8B int8 linears",
        "value": round(gbps, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["seconds_per_step"] * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 activations; N(0,0.02) weights quantized per channel)",
        "config": {
            "workload": "config1 W8A16 decode sweep: Llama-3-8B (K,N) in "
                        "{(4096,6144),(4096,4096),(4096,28672),(14336,4096)} x M in {1,8,32,64}",
            "weight_copies_rotated": LAYERS,
            "launches_per_step": dec["launches_per_step"],
            "bytes_per_step": dec["bytes_per_step"],
        },
        "roofline": {  # the decode launches: per-launch algorithmic bytes / average duration
            "bound": "hbm",
            "achieved": round(gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(gbps / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "traffic_unit": "HBM bytes per launch, mean over the sweep's launches",
            "traffic_source": (f"profiles/{PROFILE_TRAFFIC.name}: rocprofv3 --pmc FETCH_SIZE and "
                               "--pmc WRITE_SIZE runs of this sweep, each scaled by its reading "
                               "for a plain 64 MiB copy" if traffic is not None else why),
            "algorithmic_bytes_per_launch": round(dec["bytes_per_step"]
                                                  / dec["launches_per_step"]),
            "avg_launch_us": round(dec["seconds_per_step"] / dec["launches_per_step"] * 1e6, 3),
        },
        "cpu_baseline": cpu,
        "cpu_int8_restatements": cpu_int8,
        "decode_by_m_gbps": dec["by_m_gbps"],
        "decode_by_shape": dec["by_shape"],
        "decode_attention_projections_drop_in": dec["qkv_drop_in"],
        **secondary,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
