"""Int8 checkpoint format and loader: a quantized model on disk, loaded without ever holding its
projections in bf16.

The reference loads bf16 weights with `AutoModelForCausalLM.from_pretrained(path)`
(src/llm_serving_engine/model/model_runner.py:50-52) and its int8 switch would quantize after
that (model_runner.py:45-46). A quantized model saved here reloads straight into `Int8Linear` /
`Int8GluMLP` modules (and, in the W8A8 mode, `Int8RMSNormQuant` norms, as `quantize_model_`
sets them up): the loader builds the model skeleton on the meta device, allocates only the int8
buffers and the parameters that stay bf16 (embeddings, norms, lm_head), and packs the int8
weights on the GPU as they arrive.

Format (one safetensors file, little-endian, no pickled objects):
  * `<module>.qweight`: int8 (N, K) row-major per-output-channel weight of each quantized
    projection, `<module>.scales`: fp32 (N,), and `<module>.bias` (bf16, when the projection has
    one: `attention_bias` / `mlp_bias` configs), under the HF module names
    (`model.layers.{i}.self_attn.q_proj`, ..., `model.layers.{i}.mlp.down_proj`); a fused
    gate/up is stored as its two projections;
  * every other parameter under its HF name, bf16;
  * metadata: `format` = "lse-int8", `format_version` = "1", `mode` ("int8" or "w8a8"),
    `config` (the model's config as JSON).
"""

from __future__ import annotations

import json
from pathlib import Path

import torch
from torch import nn

from . import ops
from .int8_linear import (Int8GateUp, Int8GluMLP, Int8Linear, Int8RMSNormQuant, PackedBf16Linear,
                          group_qkv)

FORMAT = "lse-int8"
MODEL_TYPES = ("llama",)  # architectures the loader rebuilds (LlamaForCausalLM)
FORMAT_VERSION = "1"
ATTENTION = ("q_proj", "k_proj", "v_proj", "o_proj")
MLP = ("gate_proj", "up_proj", "down_proj")


def _check_model_type(model_type: str | None) -> None:
    if model_type not in MODEL_TYPES:
        raise RuntimeError(f"int8 checkpoints rebuild {MODEL_TYPES} models, not {model_type!r}")


def _fused_mlp(config) -> bool:
    """Whether the loader rebuilds a layer's MLP as the fused `Int8GluMLP` (what
    `quantize_model_` builds for a bias-free SiLU MLP) or as three `Int8Linear` projections."""
    return not getattr(config, "mlp_bias", False) and getattr(config, "hidden_act", "silu") == "silu"


def _quantized_tensors(model: nn.Module) -> tuple[dict[str, torch.Tensor], str]:
    """name -> CPU tensor for every quantized projection (weight, scales and bias when present),
    and the model's mode."""
    out: dict[str, torch.Tensor] = {}
    modes = set()

    def put(prefix: str, mod: Int8Linear) -> None:
        out[f"{prefix}.qweight"] = mod.unpacked_qweight().cpu()
        out[f"{prefix}.scales"] = mod.scales.cpu()
        if mod.bias is not None:
            out[f"{prefix}.bias"] = mod.bias.detach().to(torch.bfloat16).cpu().contiguous()
        modes.add(mod.mode)

    for i, layer in enumerate(model.model.layers):
        prefix = f"model.layers.{i}"
        for name in ATTENTION:
            mod = getattr(layer.self_attn, name)
            if not isinstance(mod, Int8Linear):
                raise RuntimeError(f"{prefix}.self_attn.{name} is not quantized")
            put(f"{prefix}.self_attn.{name}", mod)
        mlp = layer.mlp
        if isinstance(mlp, Int8GluMLP):
            gu = mlp.gate_up
            q, s, inter = gu.unpacked_qweight().cpu(), gu.scales.cpu(), gu.intermediate_size
            for name, (q_part, s_part) in (("gate_proj", (q[:inter], s[:inter])),
                                           ("up_proj", (q[inter:], s[inter:]))):
                out[f"{prefix}.mlp.{name}.qweight"] = q_part.contiguous()
                out[f"{prefix}.mlp.{name}.scales"] = s_part.contiguous()
            modes.add(gu.mode)
            put(f"{prefix}.mlp.down_proj", mlp.down_proj)
        else:
            for name in MLP:
                mod = getattr(mlp, name)
                if not isinstance(mod, Int8Linear):
                    raise RuntimeError(f"{prefix}.mlp.{name} is not quantized")
                put(f"{prefix}.mlp.{name}", mod)
    if len(modes) != 1:
        raise RuntimeError(f"mixed quantization modes {sorted(modes)}")
    return out, modes.pop()


def save_int8_checkpoint(model: nn.Module, path: str | Path) -> Path:
    """Writes a model quantized by `quantize_model_` to `path` (a .safetensors file)."""
    from safetensors.torch import save_file

    _check_model_type(getattr(model.config, "model_type", None))
    tensors, mode = _quantized_tensors(model)
    tied = getattr(model.config, "tie_word_embeddings", False)
    state = model.state_dict()
    head = getattr(model, "lm_head", None)
    if isinstance(head, PackedBf16Linear):  # stored row-major, as an unquantized lm_head is
        state.pop("lm_head.wp")
        if not tied:
            state["lm_head.weight"] = head.unpacked_weight()
    for name, t in state.items():
        if t.is_floating_point() and not name.endswith((".qweight", ".scales")):
            owner = name.rsplit(".", 1)[0]
            if any(owner.endswith(f".{p}") for p in ATTENTION + MLP) or ".gate_up." in name:
                continue
            if name.endswith("lm_head.weight") and tied:
                continue  # tied to embed_tokens.weight
            tensors[name] = t.detach().to(torch.bfloat16).cpu().contiguous()
    meta = {"format": FORMAT, "format_version": FORMAT_VERSION, "mode": mode,
            "config": model.config.to_json_string()}
    path = Path(path)
    save_file(tensors, str(path), metadata=meta)
    return path


def read_metadata(path: str | Path) -> dict[str, str]:
    """The checkpoint's metadata, checked to be this format."""
    from safetensors import safe_open

    with safe_open(str(path), framework="pt") as f:
        meta = f.metadata() or {}
    if meta.get("format") != FORMAT:
        raise RuntimeError(f"{path} is not an {FORMAT} checkpoint (format={meta.get('format')!r})")
    if meta.get("format_version") != FORMAT_VERSION:
        raise RuntimeError(f"{path}: unsupported format_version {meta.get('format_version')!r}")
    return meta


def _materialize_meta(model: nn.Module, device: torch.device) -> None:
    for mod in model.modules():
        for name, p in list(mod._parameters.items()):
            if p is not None and p.is_meta:
                mod._parameters[name] = nn.Parameter(torch.empty_like(p, device=device),
                                                     requires_grad=False)
        for name, b in list(mod._buffers.items()):
            if b is not None and b.is_meta:
                mod._buffers[name] = torch.empty_like(b, device=device)


@torch.no_grad()
def load_int8_checkpoint(path: str | Path, device: torch.device | str = "cuda",
                         pack_lm_head: bool = True) -> nn.Module:
    """A `LlamaForCausalLM` with int8 projections from a checkpoint written by
    `save_int8_checkpoint`. bf16 projection weights are never allocated: the skeleton is built
    on the meta device and the int8 buffers are filled (and packed) on `device`. With
    `pack_lm_head` the lm_head becomes `PackedBf16Linear`, as `quantize_model_` leaves it."""
    from safetensors import safe_open
    from transformers import AutoConfig, LlamaForCausalLM

    meta = read_metadata(path)
    mode = meta["mode"]
    cfg_dict = json.loads(meta["config"])
    _check_model_type(cfg_dict.get("model_type"))
    config = AutoConfig.for_model(**cfg_dict)
    device = torch.device(device)
    with torch.device("meta"):
        model = LlamaForCausalLM._from_config(config, dtype=torch.bfloat16)
    model.eval()
    hidden, inter = config.hidden_size, config.intermediate_size
    fused = _fused_mlp(config)
    with safe_open(str(path), framework="pt", device="cpu") as f:
        keys = set(f.keys())

        def load_q(name: str) -> tuple[torch.Tensor, torch.Tensor]:
            return (f.get_tensor(f"{name}.qweight").to(device),
                    f.get_tensor(f"{name}.scales").to(device))

        def linear(name: str) -> Int8Linear:
            q, s = load_q(name)
            bias = f.get_tensor(f"{name}.bias").to(device) if f"{name}.bias" in keys else None
            return Int8Linear.from_quantized(q, s, mode, bias)

        for i, layer in enumerate(model.model.layers):
            prefix = f"model.layers.{i}"
            for name in ATTENTION:
                setattr(layer.self_attn, name, linear(f"{prefix}.self_attn.{name}"))
            group_qkv(layer.self_attn)  # as quantize_model_ leaves them by default
            if fused:
                qg, sg = load_q(f"{prefix}.mlp.gate_proj")
                qu, su = load_q(f"{prefix}.mlp.up_proj")
                gate_up = Int8GateUp.from_quantized(torch.cat([qg, qu]), torch.cat([sg, su]),
                                                    mode)
                del qg, qu
                layer.mlp = Int8GluMLP(gate_up, linear(f"{prefix}.mlp.down_proj"))
                assert gate_up.in_features == hidden and gate_up.intermediate_size == inter
            else:  # the config's own MLP (act_fn, biases) around three int8 projections
                for name in MLP:
                    setattr(layer.mlp, name, linear(f"{prefix}.mlp.{name}"))
        # Everything still on the meta device is a bf16 parameter or buffer of the checkpoint,
        # or a buffer computed at construction (the rotary frequencies), rebuilt below. Only
        # those are materialized: the int8 buffers above stay as loaded.
        _materialize_meta(model, device)
        names = {n for n in keys if not n.endswith((".qweight", ".scales"))}
        for name, p in list(model.named_parameters()) + list(model.named_buffers()):
            if name in names:
                p.copy_(f.get_tensor(name).to(p.dtype))
    if getattr(config, "tie_word_embeddings", False):
        model.tie_weights()
    rope = model.model.rotary_emb
    model.model.rotary_emb = type(rope)(config=config, device=device)
    if mode == "w8a8":  # as quantize_model_ does by default for this mode
        for layer in model.model.layers:
            for name in ("input_layernorm", "post_attention_layernorm"):
                setattr(layer, name, Int8RMSNormQuant(getattr(layer, name)))
    if pack_lm_head and isinstance(model.lm_head, nn.Linear) and model.lm_head.bias is None:
        model.lm_head = PackedBf16Linear.from_linear(model.lm_head)
    ops._require(all(not p.is_meta for p in model.parameters()), "parameters left on meta")
    return model
