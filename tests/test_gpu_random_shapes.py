"""Seeded random shapes through the public ops in both modes, covering every route the dispatch
picks (decode kernel and its split / wide / stationary-slice routes, the tiled kernel's tiles,
bulk-and-tail launches, K splits, the ping-pong 256 x 256 tile, staged and direct output stores):
W8A8 accumulators exactly against an fp64 GEMM on the GPU and outputs against the oracle's
epilogue, the output without the int32 result equal to the one with it; W8A16 against the
oracle's fp64 golden under the north-star tolerance (max-abs <= 1e-2 max|golden|, elementwise
rel <= 1e-2 where |golden| > 1e-3 max|golden|)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bf16_bits, to_bf16_tensor
from oracle import numerics as ora

pytestmark = pytest.mark.gpu


def _shapes(seed: int, count: int, m_max: int, n_max: int, k_max: int):
    rng = np.random.default_rng(seed)
    out = []
    # token counts spread over the dispatch classes: <= 16, 17..64, 65..256, 257..1024, more
    bounds = [(lo, min(hi, m_max)) for lo, hi in
              [(1, 16), (17, 64), (65, 256), (257, 1024), (1025, m_max)] if lo <= m_max]
    for i in range(count):
        lo, hi = bounds[i % len(bounds)]
        m = int(rng.integers(lo, hi + 1))
        n = int(rng.integers(1, n_max + 1))
        k = 16 * int(rng.integers(1, k_max // 16 + 1))
        out.append((m, n, k))
    return out


W8A8_SHAPES = _shapes(8801, 40, 3000, 20000, 4096)
W8A16_SHAPES = _shapes(8802, 30, 700, 3000, 2048)


@pytest.mark.parametrize("m,n,k", W8A8_SHAPES)
def test_w8a8_random_shapes(pkg, dev, m, n, k):
    x_bits, w = ora.seeded_inputs(9000 + m + n + k, m, n, k, outliers=True)
    q, s = pkg.ops.quantize_weight_per_channel(torch.from_numpy(w).to(dev))
    del w
    qp = pkg.ops.pack_weight(q)
    xq, sx = pkg.ops.quantize_act_per_token(to_bf16_tensor(x_bits, dev))
    y_only, _ = pkg.ops.w8a8_gemm(xq, sx, qp, s, want_acc=False, want_y=True)
    y, acc = pkg.ops.w8a8_gemm(xq, sx, qp, s, want_acc=True, want_y=True)
    exact = (xq.double() @ q.double().t()).round().to(torch.int64)
    assert torch.equal(acc.to(torch.int64), exact), f"M={m} N={n} K={k}"
    assert torch.equal(y_only, y), f"M={m} N={n} K={k}"
    y_ref = ora.w8a8_epilogue(acc.cpu().numpy(), sx.cpu().numpy(), s.cpu().numpy())
    np.testing.assert_array_equal(bf16_bits(y), y_ref, err_msg=f"M={m} N={n} K={k}")


@pytest.mark.parametrize("m,n,k", W8A16_SHAPES)
def test_w8a16_random_shapes(pkg, dev, m, n, k):
    x_bits, w = ora.seeded_inputs(9500 + m + n + k, m, n, k)
    q, s = ora.quantize_weight_per_channel(w)
    qt = pkg.ops.pack_weight(torch.from_numpy(q).to(dev))
    y = pkg.ops.w8a16_linear(to_bf16_tensor(x_bits, dev), qt, torch.from_numpy(s).to(dev))
    torch.cuda.synchronize()
    ok, msg = ora.within_tolerance(bf16_bits(y), ora.w8a16_golden(x_bits, q, s))
    assert ok, f"M={m} N={n} K={k}: {msg}"
