"""Swaps a loaded Llama-family model's projections for `Int8Linear`, in place.

This is the work the reference's int8 switch stands in for: `ModelRunner.__init__` raises
`NotImplementedError("int8 weight-only quantization")` before loading
(src/llm_serving_engine/model/model_runner.py:45-46). The swap has to finish inside
`ModelRunner.__init__`, after `from_pretrained(...).to(device)` (model_runner.py:50-52) and
before any CUDA graph is captured (engine.py:94-106), because a graph freezes kernels and
tensor addresses. lm_head stays bf16, as the reference's `emit_owed` computes it
(model_runner.py:306-307), but moves to the packed bf16 tile layout (`PackedBf16Linear`), whose
kernels stream it faster than the vendor BLAS at decode batch sizes.
"""

from __future__ import annotations

import gc

import torch
from torch import nn

from .int8_linear import (MODES, Int8GluMLP, Int8Linear, Int8RMSNormQuant, PackedBf16Linear,
                          fusable_mlp, group_qkv)

ATTENTION_PROJECTIONS = ("q_proj", "k_proj", "v_proj", "o_proj")
MLP_PROJECTIONS = ("gate_proj", "up_proj", "down_proj")


def check_int8_support(model: nn.Module) -> None:
    """Load-time refusal, in the manner of `check_custom_kernel_support`
    (model_runner.py:77-94): a Llama-family layout on a GPU in bf16."""
    if not hasattr(model, "model") or not hasattr(model.model, "layers"):
        raise RuntimeError(
            f"int8 quantization assumes a Llama-family decoder (model.model.layers); "
            f"{type(model).__name__} has no such attribute"
        )
    p = next(model.parameters())
    if p.device.type != "cuda":
        raise RuntimeError(f"int8 kernels need a CUDA (HIP) device, got {p.device}")
    if p.dtype != torch.bfloat16:
        raise RuntimeError(f"int8 kernels compute in bfloat16, the model is {p.dtype}")


@torch.no_grad()
def quantize_model_(model: nn.Module, mode: str = "int8", fuse_mlp: bool = True,
                    fuse_norm: bool | None = None, fuse_qkv: bool = True,
                    pack_lm_head: bool = True) -> nn.Module:
    """Replaces q/k/v/o of every decoder layer by `Int8Linear` (per-channel int8 weights
    quantized on the GPU) and its MLP by `Int8GluMLP` (fused gate/up + SiLU-mul, then down), or,
    with `fuse_mlp=False` or an MLP of another form, gate/up/down by `Int8Linear` each. With
    `fuse_qkv` the layer's q, k and v projections share one stacked weight (`QKVGroup`): the
    three module calls the runner makes on one input run as one GEMM. In the W8A8 mode
    (`fuse_norm`, default on for "w8a8") the layer's two RMSNorms become `Int8RMSNormQuant`,
    which quantizes the normed rows once for all their projections. With `pack_lm_head` a bf16
    `lm_head` without bias becomes `PackedBf16Linear` (same bf16 values, tile layout; a tied
    lm_head keeps its embedding and adds the packed copy). Returns the same model object."""
    if mode not in MODES:
        raise ValueError(f"mode must be one of {MODES}, got {mode!r}")
    if fuse_norm is None:
        fuse_norm = mode == "w8a8"
    if fuse_norm and mode != "w8a8":
        raise ValueError("fuse_norm feeds pre-quantized rows to W8A8 projections only")
    check_int8_support(model)
    for layer in model.model.layers:
        swaps = [(layer.self_attn, ATTENTION_PROJECTIONS)]
        if fuse_mlp and fusable_mlp(layer.mlp):
            layer.mlp = Int8GluMLP.from_mlp(layer.mlp, mode)
        else:
            swaps.append((layer.mlp, MLP_PROJECTIONS))
        for parent, names in swaps:
            for name in names:
                linear = getattr(parent, name)
                if isinstance(linear, nn.Linear):
                    setattr(parent, name, Int8Linear.from_linear(linear, mode))
                    del linear
        if fuse_qkv:
            group_qkv(layer.self_attn)
        if fuse_norm:
            for name in ("input_layernorm", "post_attention_layernorm"):
                norm = getattr(layer, name)
                if not isinstance(norm, Int8RMSNormQuant):
                    setattr(layer, name, Int8RMSNormQuant(norm))
    head = getattr(model, "lm_head", None)
    if (pack_lm_head and isinstance(head, nn.Linear) and head.bias is None
            and head.weight.dtype == torch.bfloat16):
        model.lm_head = PackedBf16Linear.from_linear(head)
        del head
    gc.collect()
    torch.cuda.empty_cache()
    return model
