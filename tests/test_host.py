"""Host-side logic without a GPU: the config switch, the module's buffers and its load-time
refusals (mirroring the reference's int8 switch, config.py:32, and the RuntimeErrors of
check_custom_kernel_support, model_runner.py:77-94)."""

from __future__ import annotations

import pytest
import torch
from torch import nn


def test_config_reads_the_reference_env_names(pkg, monkeypatch):
    monkeypatch.setenv("LLM_QUANTIZE", "int8")
    monkeypatch.setenv("LLM_DTYPE", "bfloat16")
    monkeypatch.setenv("LLM_USE_CUDA_GRAPHS", "0")
    cfg = pkg.ModelConfig.from_env()
    assert (cfg.quantize, cfg.dtype, cfg.use_cuda_graphs) == ("int8", "bfloat16", False)
    cfg.validate_quantize()


def test_config_defaults_match_the_reference(pkg):
    cfg = pkg.ModelConfig()
    assert cfg.quantize == "none" and cfg.dtype == "float16" and cfg.device == "cuda"
    cfg.validate_quantize()


def test_config_refuses_unknown_mode_and_non_bf16(pkg):
    with pytest.raises(ValueError):
        pkg.ModelConfig(quantize="int4").validate_quantize()
    with pytest.raises(RuntimeError, match="bfloat16"):
        pkg.ModelConfig(quantize="int8", dtype="float16").validate_quantize()


def test_int8_linear_holds_buffers_not_parameters(pkg):
    mod = pkg.Int8Linear(64, 32, mode="w8a8", bias=True)
    assert list(mod.parameters()) == []
    names = dict(mod.named_buffers())
    assert names["qweight"].dtype == torch.int8 and names["qweight"].shape == (2, 1, 1024)
    assert names["scales"].dtype == torch.float32 and names["scales"].shape == (32,)
    assert names["bias"].dtype == torch.bfloat16
    assert "mode=w8a8" in repr(mod)
    with pytest.raises(ValueError):
        pkg.Int8Linear(64, 32, mode="fp8")


def test_state_dict_round_trip(pkg):
    a = pkg.Int8Linear(32, 16)
    a.qweight.random_(-127, 128)
    a.scales.uniform_()
    b = pkg.Int8Linear(32, 16)
    b.load_state_dict(a.state_dict())
    assert torch.equal(a.qweight, b.qweight) and torch.equal(a.scales, b.scales)


def test_cpu_forward_fails_loudly(pkg):
    mod = pkg.Int8Linear(32, 16)
    with pytest.raises(RuntimeError, match="CUDA"):
        mod(torch.zeros(2, 32, dtype=torch.bfloat16))


def test_from_linear_refuses_cpu_weights(pkg):
    with pytest.raises(RuntimeError, match="CUDA"):
        pkg.Int8Linear.from_linear(nn.Linear(32, 16, bias=False))


def test_quantize_model_refuses_non_llama_and_cpu(pkg):
    with pytest.raises(RuntimeError, match="Llama"):
        pkg.quantize_model_(nn.Sequential(nn.Linear(16, 16)))

    from transformers import LlamaConfig, LlamaForCausalLM

    config = LlamaConfig(
        vocab_size=32, hidden_size=32, intermediate_size=64, num_hidden_layers=1,
        num_attention_heads=4, num_key_value_heads=2,
    )
    model = LlamaForCausalLM(config)
    with pytest.raises(RuntimeError, match="CUDA"):
        pkg.quantize_model_(model)
    with pytest.raises(ValueError):
        pkg.quantize_model_(model, mode="int4")


def test_ops_refuse_wrong_dtypes_before_touching_the_device(pkg):
    x = torch.zeros(2, 32, dtype=torch.float16)
    q = torch.zeros(16, 32, dtype=torch.int8)
    s = torch.ones(16)
    with pytest.raises(RuntimeError, match="CUDA"):
        pkg.ops.w8a16_linear(x, q, s)


def test_unpack_inverts_the_oracle_packing(pkg):
    """The module's host-side unpack (torch views) against the oracle's packing, with padding."""
    import numpy as np

    from oracle import numerics as ora

    rng = np.random.default_rng(4)
    for n, k in ((1, 16), (37, 80), (64, 256)):
        q = rng.integers(-127, 128, (n, k)).astype(np.int8)
        qp = torch.from_numpy(ora.pack_weight(q))
        assert tuple(qp.shape) == pkg.ops.packed_shape(n, k)
        np.testing.assert_array_equal(pkg.ops.unpack_weight(qp, n, k).numpy(), q)


def test_unpack_bf16_inverts_the_oracle_packing(pkg):
    """The packed lm_head's host-side unpack (torch views) against the oracle's bf16 packing,
    with padding rows and K columns."""
    import numpy as np

    from oracle import numerics as ora

    rng = np.random.default_rng(5)
    for n, k in ((1, 16), (37, 80), (64, 256)):
        w = rng.integers(0, 1 << 16, (n, k)).astype(np.uint16)
        wp = torch.from_numpy(ora.pack_bf16_weight(w).view(np.int16)).view(torch.bfloat16)
        wp = wp.reshape(pkg.ops.packed_bf16_shape(n, k))
        got = pkg.ops.unpack_bf16_weight(wp, n, k).view(torch.int16).numpy().view(np.uint16)
        np.testing.assert_array_equal(got, w)


def test_unpack_glu_inverts_the_oracle_packing(pkg):
    import numpy as np

    from oracle import numerics as ora

    rng = np.random.default_rng(6)
    for i, k in ((1, 16), (20, 80), (48, 256)):
        q = rng.integers(-127, 128, (2 * i, k)).astype(np.int8)
        qp = torch.from_numpy(ora.pack_glu(q))
        assert tuple(qp.shape) == pkg.ops.packed_glu_shape(i, k)
        np.testing.assert_array_equal(pkg.ops.unpack_glu(qp, i, k).numpy(), q)


def test_mlp_fusion_eligibility(pkg):
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaMLP

    from llm_serving_engine_amd.int8_linear import fusable_mlp

    assert fusable_mlp(LlamaMLP(LlamaConfig(hidden_size=32, intermediate_size=64)))
    assert not fusable_mlp(LlamaMLP(LlamaConfig(hidden_size=32, intermediate_size=64,
                                                hidden_act="gelu")))
    assert not fusable_mlp(LlamaMLP(LlamaConfig(hidden_size=32, intermediate_size=64,
                                                mlp_bias=True)))
    assert not fusable_mlp(nn.Linear(4, 4))


def _cpu_int8_llama(pkg, fused: bool):
    """A tiny Llama whose projections are CPU int8 modules (zeros; no kernel calls)."""
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(vocab_size=32, hidden_size=32, intermediate_size=64, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2)
    model = LlamaForCausalLM(cfg).to(torch.bfloat16)
    for layer in model.model.layers:
        a = layer.self_attn
        for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
            lin = getattr(a, name)
            setattr(a, name, pkg.Int8Linear(lin.in_features, lin.out_features, "int8", device="cpu"))
        if fused:
            layer.mlp = pkg.Int8GluMLP(pkg.Int8GateUp(32, 64, "int8", device="cpu"),
                                       pkg.Int8Linear(64, 32, "int8", device="cpu"))
        else:
            for name, (k, n) in (("gate_proj", (32, 64)), ("up_proj", (32, 64)),
                                 ("down_proj", (64, 32))):
                setattr(layer.mlp, name, pkg.Int8Linear(k, n, "int8", device="cpu"))
    return model


@pytest.mark.parametrize("fused", [True, False])
def test_checkpoint_layout(pkg, tmp_path, fused):
    """Tensor names, dtypes and shapes of the int8 checkpoint format, and its metadata."""
    import json

    from safetensors import safe_open

    from llm_serving_engine_amd import checkpoint

    path = pkg.save_int8_checkpoint(_cpu_int8_llama(pkg, fused), tmp_path / "m.safetensors")
    meta = checkpoint.read_metadata(path)
    assert meta["mode"] == "int8" and json.loads(meta["config"])["hidden_size"] == 32
    with safe_open(str(path), "pt") as f:
        keys = set(f.keys())
        q = f.get_tensor("model.layers.1.mlp.up_proj.qweight")
        assert q.dtype == torch.int8 and tuple(q.shape) == (64, 32)
        s = f.get_tensor("model.layers.0.self_attn.k_proj.scales")
        assert s.dtype == torch.float32 and tuple(s.shape) == (16,)
        assert f.get_tensor("model.norm.weight").dtype == torch.bfloat16
    assert "lm_head.weight" in keys and "model.embed_tokens.weight" in keys
    assert not any(k.endswith("proj.weight") or ".gate_up." in k for k in keys)


def test_checkpoint_reader_refuses_other_files(pkg, tmp_path):
    from safetensors.torch import save_file

    from llm_serving_engine_amd import checkpoint

    save_file({"x": torch.zeros(2)}, str(tmp_path / "plain.safetensors"))
    with pytest.raises(RuntimeError, match="not an lse-int8 checkpoint"):
        checkpoint.read_metadata(tmp_path / "plain.safetensors")
    save_file({"x": torch.zeros(2)}, str(tmp_path / "v9.safetensors"),
              metadata={"format": "lse-int8", "format_version": "9"})
    with pytest.raises(RuntimeError, match="format_version"):
        checkpoint.read_metadata(tmp_path / "v9.safetensors")


def test_checkpoint_refuses_architectures_it_cannot_rebuild(pkg, tmp_path):
    """The loader rebuilds LlamaForCausalLM only: saving or loading another model type (a Qwen2
    config the reference's AutoModelForCausalLM would load, say) raises instead of silently
    dropping what the Llama skeleton lacks."""
    import json

    from safetensors.torch import save_file

    from llm_serving_engine_amd import checkpoint

    model = _cpu_int8_llama(pkg, True)
    model.config.model_type = "qwen2"
    with pytest.raises(RuntimeError, match="rebuild"):
        pkg.save_int8_checkpoint(model, tmp_path / "q.safetensors")
    save_file({"x": torch.zeros(2)}, str(tmp_path / "q2.safetensors"),
              metadata={"format": "lse-int8", "format_version": "1", "mode": "int8",
                        "config": json.dumps({"model_type": "qwen2"})})
    with pytest.raises(RuntimeError, match="rebuild"):
        checkpoint.load_int8_checkpoint(tmp_path / "q2.safetensors", "cpu")


def test_checkpoint_stores_projection_biases(pkg, tmp_path):
    from safetensors import safe_open

    model = _cpu_int8_llama(pkg, False)
    lin = pkg.Int8Linear(32, 32, "int8", bias=True, device="cpu")
    lin.bias.fill_(0.25)
    model.model.layers[0].self_attn.o_proj = lin
    path = pkg.save_int8_checkpoint(model, tmp_path / "b.safetensors")
    with safe_open(str(path), "pt") as f:
        b = f.get_tensor("model.layers.0.self_attn.o_proj.bias")
        assert b.dtype == torch.bfloat16 and torch.all(b == 0.25)
        assert "model.layers.1.self_attn.o_proj.bias" not in set(f.keys())
