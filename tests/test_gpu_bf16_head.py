"""bf16 decode GEMM (the lm_head the int8 path keeps in bf16: `emit_owed`,
src/llm_serving_engine/model/model_runner.py:306-307) on the GPU, through the C ABI.

Tolerance: the W8A16 rule (max-abs <= 1e-2 max|golden|, rel <= 1e-2 where |golden| >
1e-3 max|golden|) against an fp64 golden (small shapes) or the fp32 GPU product (the full
lm_head shape, whose fp64 CPU product would take minutes).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bf16_bits, to_bf16_tensor
from oracle import numerics as ora

pytestmark = pytest.mark.gpu


def test_pack_bit_exact(pkg, dev):
    rng = np.random.default_rng(2)
    for n, k in ((1, 16), (37, 80), (300, 1040)):
        w = ora.f32_to_bf16_bits(rng.standard_normal((n, k), dtype=np.float32))
        wp = pkg.ops.pack_bf16_weight(to_bf16_tensor(w, dev))
        got = wp.cpu().view(torch.int16).numpy().view(np.uint16)
        np.testing.assert_array_equal(got.reshape(-1), ora.pack_bf16_weight(w).reshape(-1))


@pytest.mark.parametrize("m", [1, 2, 8, 16, 17, 32, 33, 48, 64])
@pytest.mark.parametrize("n,k", [(1000, 1040), (100, 64), (33, 4096 + 48)])
def test_matches_the_oracle(pkg, dev, m, n, k):
    rng = np.random.default_rng(m + n + k)
    x = ora.f32_to_bf16_bits(rng.standard_normal((m, k), dtype=np.float32))
    w = ora.f32_to_bf16_bits(rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    wp = pkg.ops.pack_bf16_weight(to_bf16_tensor(w, dev))
    y = bf16_bits(pkg.ops.bf16_decode_linear(to_bf16_tensor(x, dev), wp, n))
    ok, msg = ora.within_tolerance(y, ora.bf16_linear_golden(x, w))
    assert ok, f"M={m} N={n} K={k}: {msg}"


@pytest.mark.parametrize("m", [17, 32, 33, 64, 65, 200])
def test_tiles_match_the_oracle(pkg, dev, m):
    """17..64 tokens over at least 1024 row tiles (the lm_head's class) and every M above 64 run
    as bf16 tiles of the tiled kernel; N = 16400 is 1025 row tiles, and 16400 % 128 leaves a
    partial last column tile."""
    n, k = 16400, 1040
    rng = np.random.default_rng(m)
    x = ora.f32_to_bf16_bits(rng.standard_normal((m, k), dtype=np.float32))
    w = ora.f32_to_bf16_bits(rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    wp = pkg.ops.pack_bf16_weight(to_bf16_tensor(w, dev))
    y = bf16_bits(pkg.ops.bf16_decode_linear(to_bf16_tensor(x, dev), wp, n))
    ok, msg = ora.within_tolerance(y, ora.bf16_linear_golden(x, w))
    assert ok, f"M={m}: {msg}"


@pytest.mark.parametrize("m", [1, 32, 64])
def test_llama3_lm_head_shape(pkg, dev, m):
    """N = 128256, K = 4096 against the fp32 product on the GPU and torch's bf16 F.linear."""
    g = torch.Generator(device="cpu").manual_seed(m)
    w = (torch.randn(128256, 4096, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    x = torch.randn(m, 4096, generator=g).to(torch.bfloat16).to(dev)
    y = pkg.ops.bf16_decode_linear(x, pkg.ops.pack_bf16_weight(w), 128256)
    ref = (x.float() @ w.float().t()).double().cpu().numpy()
    ok, msg = ora.within_tolerance(bf16_bits(y), ref)
    assert ok, msg
    blas = torch.nn.functional.linear(x, w)
    assert (y.float() - blas.float()).abs().max().item() <= 1e-2 * ref.__abs__().max()


@pytest.mark.parametrize("n", [3000, 16400])
def test_batch_invariant_and_deterministic(pkg, dev, n):
    """Inside each token class a row's bits do not depend on M: the decode kernel's classes over
    a narrow weight (3000 rows), the bf16 tiles' over a wide one (16400 rows, 1025 row tiles),
    and beyond 64 tokens."""
    g = torch.Generator(device="cpu").manual_seed(9)
    w = (torch.randn(n, 2048, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    x = torch.randn(200, 2048, generator=g).to(torch.bfloat16).to(dev)
    wp = pkg.ops.pack_bf16_weight(w)
    full = pkg.ops.bf16_decode_linear(x, wp, n)
    for lo, hi in ((1, 16), (17, 32), (33, 64), (65, 200)):
        part = pkg.ops.bf16_decode_linear(x[:lo], wp, n)
        assert torch.equal(part, pkg.ops.bf16_decode_linear(x[:hi], wp, n)[:lo])
    assert torch.equal(full, pkg.ops.bf16_decode_linear(x, wp, n))
