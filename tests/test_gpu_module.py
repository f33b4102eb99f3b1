"""`Int8Linear` as the engine sees it: an `nn.Linear(bias=False)` replacement on the current
stream, capturable into a CUDA (HIP) graph, swapped into a Llama model by `quantize_model_`."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

from helpers import bf16_bits
from oracle import numerics as ora

pytestmark = pytest.mark.gpu


def _linear(dev, k, n, seed, bias=False):
    torch.manual_seed(seed)
    lin = nn.Linear(k, n, bias=bias, dtype=torch.bfloat16, device=dev)
    nn.init.normal_(lin.weight, std=0.02)
    return lin


@pytest.mark.parametrize("mode", ["int8", "w8a8"])
@pytest.mark.parametrize("shape", [(1, 1, 256), (1, 7, 256), (1, 96, 256), (3, 5, 256)])
def test_forward_matches_oracle(pkg, dev, mode, shape):
    lin = _linear(dev, 256, 192, 0)
    mod = pkg.Int8Linear.from_linear(lin, mode)
    assert isinstance(mod.qweight, torch.Tensor) and not isinstance(mod.qweight, nn.Parameter)
    x = torch.randn(*shape, device=dev).to(torch.bfloat16)
    y = mod(x)
    assert y.shape == (*shape[:-1], 192) and y.dtype == torch.bfloat16
    q_ref, s_ref = ora.quantize_weight_per_channel(lin.weight.detach().float().cpu().numpy())
    np.testing.assert_array_equal(mod.unpacked_qweight().cpu().numpy(), q_ref)
    np.testing.assert_array_equal(mod.qweight.cpu().numpy(), ora.pack_weight(q_ref))
    np.testing.assert_array_equal(mod.scales.cpu().numpy(), s_ref)
    x_bits = bf16_bits(x.reshape(-1, 256))
    if mode == "int8":
        ok, msg = ora.within_tolerance(bf16_bits(y.reshape(-1, 192)), ora.w8a16_golden(x_bits, q_ref, s_ref))
        assert ok, msg
    else:
        xq, sx = ora.quantize_act_per_token(x_bits)
        expect = ora.w8a8_epilogue(ora.w8a8_accumulate(xq, q_ref), sx, s_ref)
        np.testing.assert_array_equal(bf16_bits(y.reshape(-1, 192)), expect)


def test_bias_is_added(pkg, dev):
    lin = _linear(dev, 64, 48, 1, bias=True)
    mod = pkg.Int8Linear.from_linear(lin)
    x = torch.randn(4, 64, device=dev).to(torch.bfloat16)
    no_bias = pkg.ops.w8a16_linear(x, mod.qweight, mod.scales)
    assert torch.equal(mod(x), no_bias + lin.bias.detach())


def test_non_contiguous_input(pkg, dev):
    lin = _linear(dev, 128, 64, 2)
    mod = pkg.Int8Linear.from_linear(lin)
    base = torch.randn(8, 256, device=dev).to(torch.bfloat16)
    x = base[:, 64:192]  # row stride 256, offset 128 bytes
    assert torch.equal(mod(x), mod(x.contiguous()))
    xt = torch.randn(128, 8, device=dev).to(torch.bfloat16).t()  # last dim strided
    assert torch.equal(mod(xt), mod(xt.contiguous()))


def test_runs_on_the_current_stream_and_captures_into_a_graph(pkg, dev):
    """Graph replay equals eager bitwise, replay after replay, with eager work between them."""
    lin = _linear(dev, 512, 384, 3)
    mods = [pkg.Int8Linear.from_linear(lin, "int8"), pkg.Int8Linear.from_linear(lin, "w8a8")]
    for mod in mods:
        static_x = torch.randn(16, 512, device=dev).to(torch.bfloat16)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                mod(static_x)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            static_y = mod(static_x)
        for i in range(4):
            static_x.copy_(torch.randn(16, 512, device=dev).to(torch.bfloat16))
            graph.replay()
            torch.cuda.synchronize()
            eager = mod(static_x)
            torch.cuda.synchronize()
            assert torch.equal(static_y, eager), f"replay {i} ({mod.mode})"


def test_quantize_model_swaps_llama_projections(pkg, dev):
    from transformers import LlamaConfig, LlamaForCausalLM

    torch.manual_seed(0)
    config = LlamaConfig(
        vocab_size=64, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
        num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64,
        bos_token_id=None, eos_token_id=None, pad_token_id=None,
    )
    model = LlamaForCausalLM(config).to(device=dev, dtype=torch.bfloat16).eval()
    ids = torch.randint(0, 64, (1, 12), device=dev)
    with torch.no_grad():
        ref_logits = model(ids).logits.float()
    head_weight = model.lm_head.weight.detach().clone()
    pkg.quantize_model_(model, "int8")
    for layer in model.model.layers:
        for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
            assert isinstance(getattr(layer.self_attn, name), pkg.Int8Linear)
        assert isinstance(layer.mlp, pkg.Int8GluMLP)
        assert isinstance(layer.mlp.gate_up, pkg.Int8GateUp)
        assert isinstance(layer.mlp.down_proj, pkg.Int8Linear)
    assert isinstance(model.lm_head, pkg.PackedBf16Linear)  # bf16, in the packed tile layout
    assert torch.equal(model.lm_head.unpacked_weight(), head_weight)
    assert next(model.parameters()).dtype == torch.bfloat16
    with torch.no_grad():
        logits = model(ids).logits.float()
    err = (logits - ref_logits).abs().max().item()
    assert err <= 0.05 * ref_logits.abs().max().item(), err


@pytest.mark.parametrize("m", [1, 24, 64, 100])
def test_packed_lm_head_is_a_drop_in(pkg, dev, m):
    """PackedBf16Linear against the bf16 nn.Linear it replaces: within the W8A16 tolerance of the
    fp64 product (both are bf16 products with fp32 sums, in different orders), the same bits as
    the op it wraps, and refusals for what it cannot hold."""
    import numpy as np

    from helpers import bf16_bits
    from oracle import numerics as ora

    g = torch.Generator(device="cpu").manual_seed(m)
    lin = nn.Linear(1040, 16400, bias=False, dtype=torch.bfloat16).to(dev)
    with torch.no_grad():
        lin.weight.copy_((torch.randn(16400, 1040, generator=g) * 0.02).to(torch.bfloat16))
    head = pkg.PackedBf16Linear.from_linear(lin)
    x = torch.randn(1, m, 1040, generator=g).to(torch.bfloat16).to(dev)
    y = head(x)
    assert y.shape == (1, m, 16400) and y.dtype == torch.bfloat16
    golden = (x[0].double() @ lin.weight.detach().double().t()).cpu().numpy()
    ok, msg = ora.within_tolerance(bf16_bits(y[0]), golden)
    assert ok, msg
    assert torch.equal(y[0], pkg.ops.bf16_decode_linear(x[0], head.wp, 16400))
    assert np.array_equal(head.unpacked_weight().cpu().view(torch.int16).numpy(),
                          lin.weight.detach().cpu().view(torch.int16).numpy())
    with pytest.raises(RuntimeError, match="bias"):
        pkg.PackedBf16Linear.from_linear(nn.Linear(64, 16, dtype=torch.bfloat16, device=dev))
    with pytest.raises(RuntimeError, match="bf16"):
        pkg.PackedBf16Linear.from_linear(nn.Linear(64, 16, bias=False, device=dev))


def test_load_time_refusals(pkg, dev):
    odd = nn.Linear(40, 16, bias=False, dtype=torch.bfloat16, device=dev)
    with pytest.raises(RuntimeError, match="in_features"):
        pkg.Int8Linear.from_linear(odd)
    fp16_model = nn.Module()
    with pytest.raises(RuntimeError, match="Llama"):
        pkg.quantize_model_(fp16_model)


def _attention_projections(pkg, dev, mode, bias=False, seed=30):
    """q (256 -> 256), k and v (256 -> 64) of one attention layer, as Int8Linear."""
    attn = nn.Module()
    for i, (name, n) in enumerate((("q_proj", 256), ("k_proj", 64), ("v_proj", 64))):
        setattr(attn, name, pkg.Int8Linear.from_linear(_linear(dev, 256, n, seed + i, bias), mode))
    return attn


@pytest.mark.parametrize("mode", ["int8", "w8a8"])
@pytest.mark.parametrize("m", [1, 40, 130])
def test_grouped_qkv_is_one_gemm_over_the_stacked_weight(pkg, dev, mode, m):
    """The three calls the runner makes (model_runner.py:322-324) on one input: the first runs
    the stacked (K, Nq + Nk + Nv) GEMM, the other two return their columns of it (no launch of
    their own: their outputs share its storage), and every module's output equals the stacked
    product's columns bitwise, with the modules' own buffers still valid packed weights."""
    from llm_serving_engine_amd.int8_linear import group_qkv

    attn = _attention_projections(pkg, dev, mode)
    separate = {n: getattr(attn, n) for n in ("q_proj", "k_proj", "v_proj")}
    unpacked = {n: mod.unpacked_qweight().clone() for n, mod in separate.items()}
    group = group_qkv(attn)
    assert group is not None and group.n == 384
    x = torch.randn(m, 256, device=dev).to(torch.bfloat16)
    q, k, v = attn.q_proj(x), attn.k_proj(x), attn.v_proj(x)
    assert q.untyped_storage().data_ptr() == k.untyped_storage().data_ptr() == \
        v.untyped_storage().data_ptr()
    stacked = (pkg.ops.w8a16_linear(x, group.qweight, group.scales) if mode == "int8"
               else pkg.ops.w8a8_linear(x, group.qweight, group.scales))
    assert torch.equal(torch.cat([q, k, v], -1), stacked)
    for n, mod in separate.items():
        assert torch.equal(mod.unpacked_qweight(), unpacked[n])  # views of the stacked weight
    assert group._out is None, "the product is released once all three took their columns"


def test_grouped_qkv_recomputes_for_a_new_or_modified_input(pkg, dev):
    from llm_serving_engine_amd.int8_linear import group_qkv

    attn = _attention_projections(pkg, dev, "int8")
    group_qkv(attn)
    x = torch.randn(5, 256, device=dev).to(torch.bfloat16)
    q = attn.q_proj(x)
    x2 = torch.randn(5, 256, device=dev).to(torch.bfloat16)
    k2 = attn.k_proj(x2)  # another input: computed afresh
    x.mul_(2.0)  # the first input modified in place: its version moved
    v = attn.v_proj(x)
    fresh_k = attn.k_proj(x2)
    assert torch.equal(k2, fresh_k)
    q_again, _, v_again = attn.q_proj(x), attn.k_proj(x), attn.v_proj(x)
    assert torch.equal(v, v_again) and not torch.equal(q, q_again)


def test_grouped_qkv_with_bias_and_in_a_graph(pkg, dev):
    from llm_serving_engine_amd.int8_linear import group_qkv

    attn = _attention_projections(pkg, dev, "int8", bias=True)
    x = torch.randn(3, 256, device=dev).to(torch.bfloat16)
    ref = [getattr(attn, n)(x) for n in ("q_proj", "k_proj", "v_proj")]
    group_qkv(attn)
    eager = [getattr(attn, n)(x) for n in ("q_proj", "k_proj", "v_proj")]
    for a, b in zip(ref, eager):  # separate and stacked launches: same tolerance class
        assert (a.float() - b.float()).abs().max() <= 2e-2 * a.float().abs().max()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = [getattr(attn, n)(x) for n in ("q_proj", "k_proj", "v_proj")]
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(eager, outs):
            assert torch.equal(a, b)


def test_quantized_llama_groups_every_layer(pkg, dev):
    """quantize_model_ groups q/k/v in every layer by default; HF LlamaAttention (three calls on
    one input, modeling_llama.py:254-256) then gives the logits of the ungrouped model up to the
    stacked launch's fp32 summation order."""
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(vocab_size=96, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64,
                      bos_token_id=None, eos_token_id=None, pad_token_id=None)
    models = []
    for fuse_qkv in (True, False):
        torch.manual_seed(5)
        with torch.device(dev):
            models.append(pkg.quantize_model_(
                LlamaForCausalLM._from_config(cfg, dtype=torch.bfloat16).eval(), "int8",
                fuse_qkv=fuse_qkv))
    grouped, plain = models
    for layer in grouped.model.layers:
        assert layer.self_attn.k_proj.__dict__.get("_qkv_group") is not None
    ids = torch.randint(0, 96, (1, 13), device=dev)
    with torch.no_grad():
        a, b = grouped(ids).logits.float(), plain(ids).logits.float()
    assert ((a - b).norm() / b.norm()) < 1e-2


def _tiny_llama(pkg, dev, mode, seed=5):
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(vocab_size=96, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64,
                      bos_token_id=None, eos_token_id=None, pad_token_id=None)
    torch.manual_seed(seed)
    with torch.device(dev):
        return pkg.quantize_model_(
            LlamaForCausalLM._from_config(cfg, dtype=torch.bfloat16).eval(), mode)


@pytest.mark.parametrize("mode", ["int8", "w8a8"])
def test_grouped_qkv_and_quantized_llama_under_inference_mode(pkg, dev, mode):
    """Serving stacks run under torch.inference_mode(), whose tensors carry no version counter:
    the grouped q/k/v still serve the three calls from one stacked GEMM, and a quantized Llama
    forward gives the same logits as under no_grad (the reference's mode)."""
    from llm_serving_engine_amd.int8_linear import group_qkv

    attn = _attention_projections(pkg, dev, mode)
    group_qkv(attn)
    with torch.inference_mode():
        x = torch.randn(7, 256, device=dev).to(torch.bfloat16)
        assert x.is_inference()
        q, k, v = attn.q_proj(x), attn.k_proj(x), attn.v_proj(x)
        assert q.untyped_storage().data_ptr() == v.untyped_storage().data_ptr()
        stacked = (pkg.ops.w8a16_linear(x, attn.q_proj.__dict__["_qkv_group"].qweight,
                                        attn.q_proj.__dict__["_qkv_group"].scales)
                   if mode == "int8" else None)
    if stacked is not None:
        assert torch.equal(torch.cat([q, k, v], -1), stacked)
    model = _tiny_llama(pkg, dev, mode)
    ids = torch.randint(0, 96, (2, 11), device=dev)
    with torch.no_grad():
        ref = model(ids).logits
    with torch.inference_mode():
        got = model(ids).logits
    assert torch.equal(got, ref)


def test_grouped_qkv_survives_a_device_round_trip(pkg, dev):
    """Module._apply (model.to(...)) replaces the grouped modules' buffers with tensors that are
    no longer views of the stacked weight; the group stacks them again and the logits do not
    change."""
    model = _tiny_llama(pkg, dev, "int8", seed=9)
    ids = torch.randint(0, 96, (1, 9), device=dev)
    with torch.no_grad():
        before = model(ids).logits
        model.to("cpu").to(dev)
        group = model.model.layers[0].self_attn.q_proj.__dict__["_qkv_group"]
        assert not group._members_are_views()
        after = model(ids).logits
    assert group._members_are_views() and group.qweight.device.type == "cuda"
    assert torch.equal(after, before)
