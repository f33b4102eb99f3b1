"""The int8 checkpoint round trip on the GPU: a quantized Llama saved and reloaded gives
bit-identical logits, and loading never allocates the bf16 projection weights."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _llama(dev, seed=0, **kw):
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = dict(vocab_size=96, hidden_size=128, intermediate_size=352, num_hidden_layers=2,
               num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64,
               bos_token_id=None, eos_token_id=None, pad_token_id=None)
    cfg.update(kw)
    torch.manual_seed(seed)
    # As from_pretrained(dtype=bfloat16) builds it: bf16 parameters, fp32 rotary frequencies
    # (a .to(dtype=bfloat16) of the whole model would round those too).
    with torch.device(dev):
        model = LlamaForCausalLM._from_config(LlamaConfig(**cfg), dtype=torch.bfloat16)
    return model.eval()


@pytest.mark.parametrize("mode", ["int8", "w8a8"])
def test_round_trip_is_bit_identical(pkg, dev, tmp_path, mode):
    model = pkg.quantize_model_(_llama(dev), mode)
    ids = torch.randint(0, 96, (1, 11), device=dev)
    with torch.no_grad():
        ref = model(ids).logits
    path = pkg.save_int8_checkpoint(model, tmp_path / "m.safetensors")
    loaded = pkg.load_int8_checkpoint(path, dev)
    assert next(loaded.parameters()).dtype == torch.bfloat16
    for layer in loaded.model.layers:
        assert isinstance(layer.mlp, pkg.Int8GluMLP)
        assert isinstance(layer.self_attn.q_proj, pkg.Int8Linear)
        assert layer.self_attn.q_proj.mode == mode
    assert isinstance(loaded.lm_head, pkg.PackedBf16Linear)
    with torch.no_grad():
        got = loaded(ids).logits
    assert torch.equal(got, ref)


def test_round_trip_with_tied_embeddings(pkg, dev, tmp_path):
    """A tied lm_head (Llama-3.2's tie_word_embeddings) is stored once, as the embedding, and
    comes back packed from it: bit-identical logits."""
    from safetensors import safe_open

    model = pkg.quantize_model_(_llama(dev, 3, tie_word_embeddings=True), "int8")
    assert isinstance(model.lm_head, pkg.PackedBf16Linear)
    assert torch.equal(model.lm_head.unpacked_weight(), model.model.embed_tokens.weight)
    ids = torch.randint(0, 96, (1, 10), device=dev)
    with torch.no_grad():
        ref = model(ids).logits
    path = pkg.save_int8_checkpoint(model, tmp_path / "t.safetensors")
    with safe_open(str(path), "pt") as f:
        assert not any(k.startswith("lm_head.") for k in f.keys())
    loaded = pkg.load_int8_checkpoint(path, dev)
    assert isinstance(loaded.lm_head, pkg.PackedBf16Linear)
    with torch.no_grad():
        got = loaded(ids).logits
    assert torch.equal(got, ref)


@pytest.mark.parametrize("mode", ["int8", "w8a8"])
def test_round_trip_keeps_projection_biases(pkg, dev, tmp_path, mode):
    """attention_bias and mlp_bias configs (transformers modeling_llama.py:169-171, 231-241):
    the biases are stored beside each projection's int8 weight and restored, the MLP stays
    unfused (the fused kernel takes bias-free projections), and logits are bit-identical."""
    from safetensors import safe_open

    base = _llama(dev, 7, attention_bias=True, mlp_bias=True)
    with torch.no_grad():
        for name, p in base.named_parameters():
            if name.endswith(".bias"):
                p.normal_(0.0, 0.5)
    model = pkg.quantize_model_(base, mode)
    ids = torch.randint(0, 96, (1, 9), device=dev)
    with torch.no_grad():
        ref = model(ids).logits
    path = pkg.save_int8_checkpoint(model, tmp_path / "b.safetensors")
    with safe_open(str(path), "pt") as f:
        biases = [k for k in f.keys() if k.endswith(".bias")]
    assert len(biases) == 2 * 7, biases  # q, k, v, o, gate, up, down in each of 2 layers
    loaded = pkg.load_int8_checkpoint(path, dev)
    for layer in loaded.model.layers:
        assert layer.self_attn.o_proj.bias is not None
        assert isinstance(layer.mlp.down_proj, pkg.Int8Linear) and layer.mlp.down_proj.bias is not None
    with torch.no_grad():
        got = loaded(ids).logits
    assert torch.equal(got, ref)


def test_unfused_model_saves_the_same_weights(pkg, dev, tmp_path):
    """A model quantized without MLP fusion stores the same tensors; it reloads fused."""
    from safetensors import safe_open

    a = pkg.save_int8_checkpoint(pkg.quantize_model_(_llama(dev, 3), "int8"), tmp_path / "a.st")
    b = pkg.save_int8_checkpoint(pkg.quantize_model_(_llama(dev, 3), "int8", fuse_mlp=False),
                                 tmp_path / "b.st")
    with safe_open(str(a), "pt") as fa, safe_open(str(b), "pt") as fb:
        assert set(fa.keys()) == set(fb.keys())
        for k in fa.keys():
            assert torch.equal(fa.get_tensor(k), fb.get_tensor(k)), k


def test_loading_never_holds_bf16_projections(pkg, dev, tmp_path):
    """Peak device memory while loading stays below what the bf16 projections alone would take
    (the reference's from_pretrained + quantize path would allocate them first)."""
    model = pkg.quantize_model_(
        _llama(dev, 5, hidden_size=1024, intermediate_size=2816, num_hidden_layers=4,
               num_attention_heads=8, num_key_value_heads=4), "int8")
    path = pkg.save_int8_checkpoint(model, tmp_path / "big.safetensors")
    del model
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    bf16_projection_bytes = 4 * 2 * (1024 * 1024 * 2 + 2 * 1024 * 512 + 3 * 1024 * 2816)
    torch.cuda.reset_peak_memory_stats(dev)
    base = torch.cuda.memory_allocated(dev)
    loaded = pkg.load_int8_checkpoint(path, dev)
    peak = torch.cuda.max_memory_allocated(dev) - base
    assert peak < bf16_projection_bytes, (peak, bf16_projection_bytes)
    assert loaded(torch.zeros(1, 4, dtype=torch.long, device=dev)).logits.isfinite().all()
