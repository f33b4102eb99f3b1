"""Writes the committed fixtures under tests/golden/ from the CPU oracle.

The reference ships no golden vectors for the int8 Linear path (its int8 switch raises,
src/llm_serving_engine/model/model_runner.py:45-46), so these fixtures are the oracle's own
outputs on small seeded inputs, frozen so that any later change to the oracle's numerics or to
the seeded input generator is caught (tests/test_oracle.py), and so the GPU tests have fixed
vectors to match (tests/test_gpu_golden.py replays them through the HIP kernels).

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle import numerics as ora  # noqa: E402


def small_cases() -> dict[str, np.ndarray]:
    """M=5 tokens, N=24 channels, K=48 (a K tail past 32, N past 16), with an all-zero weight
    row, an exact-tie row, and a zero activation row."""
    x, w = ora.seeded_inputs(424242, 5, 24, 48)
    w[3] = 0.0
    w[4, :5] = [127.0, 63.5, -1.0, 0.5, 2.5]
    w[4, 5:] = 0.0
    xo, _ = ora.seeded_inputs(424243, 5, 1, 48, outliers=True)
    xo[2] = 0
    q, s = ora.quantize_weight_per_channel(w)
    xq, sx = ora.quantize_act_per_token(xo)
    acc = ora.w8a8_accumulate(xq, q)
    return {
        "w": w, "q": q, "s": s, "x": x, "y_w8a16": ora.w8a16_golden(x, q, s),
        "xo": xo, "xq": xq, "sx": sx, "acc": acc, "y_w8a8": ora.w8a8_epilogue(acc, sx, s),
    }


def config0_digests() -> dict[str, str]:
    """SHA-256 of config 0's seeded inputs, quantized weights and bf16-rounded golden output."""
    x_bits, w = ora.seeded_inputs(0, 1, 2048, 2048)
    q, s = ora.quantize_weight_per_channel(w)
    y = ora.f64_to_bf16_bits(ora.w8a16_golden(x_bits, q, s))
    return {
        name: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
        for name, a in (("x_bits", x_bits), ("q", q), ("s", s), ("y_bits", y))
    }


if __name__ == "__main__":
    np.savez_compressed(HERE / "small_cases.npz", **small_cases())
    (HERE / "config0_digests.json").write_text(json.dumps(config0_digests(), indent=1) + "\n")
    print("wrote", HERE / "small_cases.npz", HERE / "config0_digests.json")
