"""RMSNorm fused with per-token quantization on the GPU (the W8A8 first stage folded into
LlamaRMSNorm, transformers modeling_llama.py:62-67), through the C ABI.

Parity: the kernel's quantization of its own bf16 normed rows is bit-exact against the pinned
oracle quantizer; its normed rows match the oracle RMSNorm except where the two fp32 variance
sums put x * r on opposite sides of a bf16 rounding boundary (at most 2 ulps after the weight
product, on fewer than 1e-3 of the elements).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bf16_bits, to_bf16_tensor
from oracle import numerics as ora

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m,k", [(1, 4096), (37, 4096), (5, 2048), (64, 64), (3, 14336), (9, 3072),
                                 (4, 6144), (2, 8192), (2, 8208)])
def test_matches_the_oracle(pkg, dev, m, k):
    rng = np.random.default_rng(m * 7 + k)
    x = rng.standard_normal((m, k), dtype=np.float32) * np.float32(2.0)
    x[0, :: max(1, k // 9)] *= 30.0  # outlier columns
    if m > 2:
        x[2] = 0.0  # all-zero row: h = 0, sx = 1, xq = 0
    x_bits = ora.f32_to_bf16_bits(x)
    w_bits = ora.f32_to_bf16_bits(1.0 + 0.2 * rng.standard_normal(k, dtype=np.float32))
    xq, sx, normed = pkg.ops.rmsnorm_quantize(to_bf16_tensor(x_bits, dev),
                                              to_bf16_tensor(w_bits, dev), 1e-5, want_normed=True)
    torch.cuda.synchronize()
    h = bf16_bits(normed)
    q_ref, s_ref = ora.quantize_act_per_token(h)
    np.testing.assert_array_equal(xq.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(sx.cpu().numpy(), s_ref)
    golden = ora.rmsnorm_bf16(x_bits, w_bits, 1e-5)
    diff = ora.bf16_ulps_apart(h, ora.bf16_bits_to_f32(golden).astype(np.float64))
    assert diff.max() <= 2.0 and np.mean(diff > 0) < 1e-3, (diff.max(), np.mean(diff > 0))
    if m > 2:
        assert np.all(h[2] == 0) and sx[2].item() == 1.0 and not xq[2].any()


def test_without_normed_output_gives_the_same_rows(pkg, dev):
    x = torch.randn(9, 1024, device=dev).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(1024, device=dev)).to(torch.bfloat16)
    a = pkg.ops.rmsnorm_quantize(x, w, 1e-6)
    b = pkg.ops.rmsnorm_quantize(x, w, 1e-6, want_normed=True)
    assert a[2] is None and torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_fused_norm_model_tracks_the_unfused_one(pkg, dev):
    """A W8A8 Llama with fused norms against the same model quantizing after the bf16 norms:
    identical except where a normed value differs in its last bf16 place."""
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(vocab_size=80, hidden_size=256, intermediate_size=688, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64,
                      bos_token_id=None, eos_token_id=None, pad_token_id=None)
    ids = torch.randint(0, 80, (1, 13), device=dev)
    logits = {}
    for fuse in (None, True, False):
        torch.manual_seed(0)
        model = LlamaForCausalLM(cfg).to(device=dev, dtype=torch.bfloat16).eval()
        if fuse is not None:
            pkg.quantize_model_(model, "w8a8", fuse_norm=fuse)
            for layer in model.model.layers:
                assert isinstance(layer.input_layernorm, pkg.Int8RMSNormQuant) == fuse
        with torch.no_grad():
            logits[fuse] = model(ids).logits.float()
    scale = logits[None].abs().max().item()
    assert (logits[True] - logits[False]).abs().max().item() <= 0.01 * scale
    assert (logits[True] - logits[None]).abs().max().item() <= 0.05 * scale


def test_quantized_rows_refused_by_weight_only_modules(pkg, dev):
    lin = torch.nn.Linear(64, 32, bias=False, dtype=torch.bfloat16, device=dev)
    mod = pkg.Int8Linear.from_linear(lin, "int8")
    x = torch.randn(4, 64, device=dev).to(torch.bfloat16)
    xq, sx, _ = pkg.ops.rmsnorm_quantize(x, torch.ones(64, dtype=torch.bfloat16, device=dev), 1e-6)
    with pytest.raises(RuntimeError, match="weight-only"):
        mod(pkg.QuantizedRows(xq, sx, x.shape))
