"""`Int8Linear`: the drop-in for `nn.Linear(K, N, bias=False)` on the engine's model path.

The reference calls its projections as plain modules, `attn.q_proj(normed)` and the like
(src/llm_serving_engine/model/model_runner.py:322-324, 369, 418; transformers
modeling_llama.py:175), so the replacement keeps exactly `forward(x) -> y` with x (..., K) and
y (..., N) in bf16 on the same device and the current stream. Quantized weights and scales are
buffers, not Parameters: the runner reads `model.dtype` off the first parameter
(model_runner.py:86,112) and must keep seeing bf16.

`qweight` holds the int8 weight in the packed tile layout the kernels stream (ops.pack_weight),
shape (ceil(N/16), ceil(K/64), 1024); `unpacked_qweight()` returns the row-major (N, K) matrix.

`Int8GluMLP` is the drop-in for the whole `LlamaMLP` (transformers modeling_llama.py:163-176),
which the runner calls as `layer.mlp(x)` (model_runner.py:223): its gate and up projections and
the SiLU-mul between them (`down_proj(act_fn(gate_proj(x)) * up_proj(x))`, line 175) run as one
`Int8GateUp` kernel, then `down_proj` as an `Int8Linear`.
"""

from __future__ import annotations

import torch
from torch import nn

from . import _lib, ops

MODES = ("int8", "w8a8")


class QuantizedRows:
    """The W8A8 form of a bf16 activation (..., K): int8 rows `xq` (rows, K) and per-row fp32
    scales `sx`, as `Int8RMSNormQuant` produces them. It stands where the norm's bf16 output
    stood: W8A8 projections take it as their input without quantizing again, and it answers the
    `shape`, `device` and `dtype` (that of the activation it encodes) the callers read
    (model_runner.py:319, 383-386; modeling_llama.py:251)."""

    __slots__ = ("xq", "sx", "shape", "device", "dtype")

    def __init__(self, xq: torch.Tensor, sx: torch.Tensor, shape: torch.Size,
                 dtype: torch.dtype = torch.bfloat16) -> None:
        self.xq, self.sx, self.shape = xq, sx, torch.Size(shape)
        self.device, self.dtype = xq.device, dtype


def _w8a8_input(mod: nn.Module, x) -> bool:
    if isinstance(x, QuantizedRows):
        if mod.mode != "w8a8":
            raise RuntimeError("pre-quantized rows reach a weight-only (int8) projection")
        return True
    return False


class Int8Linear(nn.Module):
    """y = x · (q · diag(s))ᵀ (+ bias). `mode` "int8" is weight-only W8A16 (the reference's own
    name for the switch, model_runner.py:46); "w8a8" adds dynamic per-token activation
    quantization and an int8 GEMM with exact int32 accumulation."""

    def __init__(
        self,
        in_features: int,
        out_features: int,
        mode: str = "int8",
        bias: bool = False,
        device: torch.device | str | None = None,
    ) -> None:
        super().__init__()
        if mode not in MODES:
            raise ValueError(f"mode must be one of {MODES}, got {mode!r}")
        self.in_features = in_features
        self.out_features = out_features
        self.mode = mode
        self.register_buffer(
            "qweight",
            torch.zeros(ops.packed_shape(out_features, in_features), dtype=torch.int8, device=device),
        )
        self.register_buffer("scales", torch.ones((out_features,), dtype=torch.float32, device=device))
        self.register_buffer(
            "bias", torch.zeros((out_features,), dtype=torch.bfloat16, device=device) if bias else None
        )

    @classmethod
    def from_linear(cls, linear: nn.Linear, mode: str = "int8") -> Int8Linear:
        """Quantizes `linear.weight` per output channel on its own (GPU) device."""
        check_linear_supported(linear)
        w = linear.weight.detach()
        mod = cls(linear.in_features, linear.out_features, mode, linear.bias is not None, w.device)
        q, s = ops.quantize_weight_per_channel(w)
        mod.qweight.copy_(ops.pack_weight(q))
        del q
        mod.scales.copy_(s)
        if linear.bias is not None:
            mod.bias.copy_(linear.bias.detach().to(torch.bfloat16))
        return mod

    @classmethod
    def from_quantized(
        cls, qweight: torch.Tensor, scales: torch.Tensor, mode: str = "int8",
        bias: torch.Tensor | None = None,
    ) -> Int8Linear:
        """Wraps already quantized row-major (N, K) int8 weights and (N,) fp32 scales (on the GPU;
        they are packed there)."""
        n, k = qweight.shape
        mod = cls(k, n, mode, bias is not None, qweight.device)
        mod.qweight.copy_(ops.pack_weight(qweight))
        mod.scales.copy_(scales)
        if bias is not None:
            mod.bias.copy_(bias.to(torch.bfloat16))
        return mod

    def unpacked_qweight(self) -> torch.Tensor:
        """The int8 weight as a row-major (N, K) matrix."""
        return ops.unpack_weight(self.qweight, self.out_features, self.in_features)

    def forward(self, x: torch.Tensor | QuantizedRows) -> torch.Tensor:
        group = self.__dict__.get("_qkv_group")
        if group is not None:
            y = group.columns(self, x)
        else:
            y = _int8_product(self.mode, x, self.qweight, self.scales, self.out_features)
        return y if self.bias is None else y + self.bias

    def extra_repr(self) -> str:
        return (
            f"in_features={self.in_features}, out_features={self.out_features}, "
            f"mode={self.mode}, bias={self.bias is not None}"
        )


def _int8_product(mode: str, x: torch.Tensor | QuantizedRows, qweight: torch.Tensor,
                  scales: torch.Tensor, n: int) -> torch.Tensor:
    """x (..., K) times a packed int8 weight of n rows, without bias, in `mode`."""
    if isinstance(x, QuantizedRows):
        if mode != "w8a8":
            raise RuntimeError("pre-quantized rows reach a weight-only (int8) projection")
        y, _ = ops.w8a8_gemm(x.xq, x.sx, qweight, scales)
        return y.view(*x.shape[:-1], n)
    if mode == "int8":
        return ops.w8a16_linear(x, qweight, scales)
    return ops.w8a8_linear(x, qweight, scales)


class QKVGroup:
    """One attention layer's q, k and v projections as one int8 GEMM over their stacked weights.

    The reference calls the three as separate modules on the same input, one after another
    (`_project_qkv`, src/llm_serving_engine/model/model_runner.py:322-324; HF LlamaAttention,
    modeling_llama.py:254-256). Separately they are three weight streams of which two (the
    (K, 1024) k and v of Llama-3-8B) are too small to fill the GPU; stacked they are one stream
    of (K, 6144). The modules keep their own buffers, which are views of the stacked packed weight
    (row tiles of the tile layout, so each slice is itself a packed weight) and of the stacked
    scales. The first of the three calls on an input computes all columns; the others return
    their columns of that result, as long as they see the very same input object, unmodified
    (same tensor version), and the result is dropped once all three have taken their columns.
    Any other call computes the stacked product afresh. Each module's output is a column view of
    the (..., Nq + Nk + Nv) product, bit-identical to what the stacked weight gives for those
    columns.

    Inference tensors (`torch.inference_mode`) carry no version counter, so for them a hit needs
    the same input object only: the input must not be rewritten in place between the three calls
    (the runner never does), and neither may any tensor be written through its data pointer (a
    HIP kernel's output) between them, which no version counter sees either.

    Moving or reloading the modules (`Module._apply`, `load_state_dict(assign=True)`) replaces
    their buffers with tensors that are no longer views of the stacked ones; the next call that
    computes the product notices and stacks the members' current buffers again."""

    def __init__(self, qweight: torch.Tensor, scales: torch.Tensor, mode: str,
                 members: list[Int8Linear]) -> None:
        self.qweight, self.scales, self.mode = qweight, scales, mode
        self.members = list(members)
        self.n = int(scales.shape[0])
        self.offsets: dict[int, tuple[int, int]] = {}
        at = 0
        for mod in members:
            self.offsets[id(mod)] = (at, at + mod.out_features)
            at += mod.out_features
        self._input = None
        self._version = -1
        self._out: torch.Tensor | None = None
        self._pending: set[int] = set()

    @staticmethod
    def _version_of(x) -> int | None:
        t = x.xq if isinstance(x, QuantizedRows) else x
        return None if t.is_inference() else t._version

    def _members_are_views(self) -> bool:
        """Whether every member's buffers are still its rows of the stacked weight and scales."""
        row = self.qweight.stride(0)
        for mod in self.members:
            a, _ = self.offsets[id(mod)]
            qw, sc = mod._buffers["qweight"], mod._buffers["scales"]
            if (qw.device != self.qweight.device or sc.device != self.scales.device
                    or qw.data_ptr() != self.qweight.data_ptr() + (a // 16) * row
                    or sc.data_ptr() != self.scales.data_ptr() + 4 * a
                    or sc.dtype != torch.float32):
                return False
        return True

    def _restack(self) -> None:
        """Stacks the members' current buffers again and makes them views of the result."""
        self.qweight = torch.cat([m._buffers["qweight"] for m in self.members])
        self.scales = torch.cat([m._buffers["scales"].float() for m in self.members])
        for m in self.members:
            a, b = self.offsets[id(m)]
            m._buffers["qweight"] = self.qweight[a // 16:b // 16]
            m._buffers["scales"] = self.scales[a:b]

    def columns(self, mod: Int8Linear, x) -> torch.Tensor:
        key = id(mod)
        hit = (self._out is not None and x is self._input and key in self._pending
               and self._version_of(x) == self._version)
        if not hit:
            if not self._members_are_views():
                self._restack()
            self._out = _int8_product(self.mode, x, self.qweight, self.scales, self.n)
            self._input, self._version = x, self._version_of(x)
            self._pending = set(self.offsets)
        out = self._out
        self._pending.discard(key)
        if not self._pending:  # all three served: release the input and the product
            self._out = self._input = None
        a, b = self.offsets[key]
        return out[..., a:b]


def group_qkv(attn: nn.Module) -> QKVGroup | None:
    """Makes `attn`'s q_proj, k_proj and v_proj (Int8Linear, one mode, one input width, row counts
    multiples of 16, biases all present or all absent) views of one stacked packed weight run by
    a `QKVGroup`. Returns the group, or None when they do not qualify (they then stay separate)."""
    mods = [getattr(attn, n, None) for n in ("q_proj", "k_proj", "v_proj")]
    if not all(isinstance(m, Int8Linear) for m in mods):
        return None
    if (len({m.mode for m in mods}) != 1 or len({m.in_features for m in mods}) != 1
            or any(m.out_features % 16 for m in mods)
            or len({m.bias is None for m in mods}) != 1):
        return None
    qweight = torch.cat([m.qweight for m in mods])  # row tiles stack: still the tile layout
    scales = torch.cat([m.scales for m in mods])
    at = 0
    for m in mods:
        rb = m.out_features // 16
        m._buffers["qweight"] = qweight[at // 16:at // 16 + rb]
        m._buffers["scales"] = scales[at:at + m.out_features]
        at += m.out_features
    group = QKVGroup(qweight, scales, mods[0].mode, mods)
    for m in mods:
        m.__dict__["_qkv_group"] = group
    return group


def check_linear_supported(linear: nn.Linear) -> None:
    """Load-time checks, raising RuntimeError as the reference's
    `check_custom_kernel_support` does (model_runner.py:77-94)."""
    w = linear.weight
    if w.device.type != "cuda":
        raise RuntimeError(f"int8 kernels need a CUDA (HIP) device, got {w.device}")
    k_align = _lib.query(_lib.Q_K_ALIGN)
    if linear.in_features % k_align:
        raise RuntimeError(
            f"int8 kernels need in_features % {k_align} == 0, got {linear.in_features}"
        )
    max_k = _lib.query(_lib.Q_MAX_K)
    if linear.in_features > max_k:
        raise RuntimeError(f"int8 kernels take in_features <= {max_k}, got {linear.in_features}")


def _is_silu(act: nn.Module) -> bool:
    # transformers' ACT2FN["silu"] is its own SiLUActivation (activations.py), calling F.silu.
    return isinstance(act, nn.SiLU) or type(act).__name__ == "SiLUActivation"


class Int8GateUp(nn.Module):
    """h = silu(x · (q_g · diag(s_g))ᵀ) * (x · (q_u · diag(s_u))ᵀ), x (..., K) → h (..., I) bf16:
    the gate and up projections of `LlamaMLP` and its SiLU-mul (modeling_llama.py:175) as one
    int8 GEMM whose epilogue applies the activation and the product in fp32 and rounds once.

    `qweight` holds the stacked (2I, K) [gate; up] weight in the gate/up layout (ops.pack_glu),
    `scales` the (2I,) [gate; up] per-channel scales."""

    def __init__(
        self,
        in_features: int,
        intermediate_size: int,
        mode: str = "int8",
        device: torch.device | str | None = None,
    ) -> None:
        super().__init__()
        if mode not in MODES:
            raise ValueError(f"mode must be one of {MODES}, got {mode!r}")
        self.in_features = in_features
        self.intermediate_size = intermediate_size
        self.mode = mode
        self.register_buffer(
            "qweight",
            torch.zeros(ops.packed_glu_shape(intermediate_size, in_features), dtype=torch.int8,
                        device=device),
        )
        self.register_buffer(
            "scales", torch.ones((2 * intermediate_size,), dtype=torch.float32, device=device))

    @classmethod
    def from_linears(cls, gate: nn.Linear, up: nn.Linear, mode: str = "int8") -> Int8GateUp:
        """Quantizes the bias-free `gate` and `up` projections per output channel."""
        for lin in (gate, up):
            check_linear_supported(lin)
            if lin.bias is not None:
                raise RuntimeError("the fused gate/up kernel takes bias-free projections")
        if gate.weight.shape != up.weight.shape:
            raise RuntimeError(
                f"gate and up shapes differ: {tuple(gate.weight.shape)} vs {tuple(up.weight.shape)}")
        q_g, s_g = ops.quantize_weight_per_channel(gate.weight.detach())
        q_u, s_u = ops.quantize_weight_per_channel(up.weight.detach())
        return cls.from_quantized(torch.cat([q_g, q_u]), torch.cat([s_g, s_u]), mode)

    @classmethod
    def from_quantized(cls, qweight: torch.Tensor, scales: torch.Tensor,
                       mode: str = "int8") -> Int8GateUp:
        """Wraps an already quantized stacked (2I, K) int8 [gate; up] weight and its (2I,) fp32
        scales (on the GPU; packed there)."""
        two_i, k = qweight.shape
        mod = cls(k, two_i // 2, mode, qweight.device)
        mod.qweight.copy_(ops.pack_glu(qweight))
        mod.scales.copy_(scales)
        return mod

    def unpacked_qweight(self) -> torch.Tensor:
        """The stacked (2I, K) int8 [gate; up] weight, row-major."""
        return ops.unpack_glu(self.qweight, self.intermediate_size, self.in_features)

    def forward(self, x: torch.Tensor | QuantizedRows) -> torch.Tensor:
        if _w8a8_input(self, x):
            h = ops.w8a8_glu_quantized(x.xq, x.sx, self.qweight, self.scales)
            return h.view(*x.shape[:-1], self.intermediate_size)
        if self.mode == "int8":
            return ops.w8a16_glu(x, self.qweight, self.scales)
        return ops.w8a8_glu(x, self.qweight, self.scales)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, intermediate_size={self.intermediate_size}, "
                f"mode={self.mode}")


class Int8GluMLP(nn.Module):
    """Drop-in for `LlamaMLP` (modeling_llama.py:163-176): forward(x) = down_proj(gate_up(x))."""

    def __init__(self, gate_up: Int8GateUp, down_proj: Int8Linear) -> None:
        super().__init__()
        self.gate_up = gate_up
        self.down_proj = down_proj

    @classmethod
    def from_mlp(cls, mlp: nn.Module, mode: str = "int8") -> Int8GluMLP:
        """Quantizes a `LlamaMLP` (gate_proj, up_proj, down_proj, SiLU act_fn, no bias)."""
        if not _is_silu(mlp.act_fn):
            raise RuntimeError(
                f"the fused gate/up kernel applies SiLU, the MLP uses {type(mlp.act_fn).__name__}")
        return cls(Int8GateUp.from_linears(mlp.gate_proj, mlp.up_proj, mode),
                   Int8Linear.from_linear(mlp.down_proj, mode))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.down_proj(self.gate_up(x))


def fusable_mlp(mlp: nn.Module) -> bool:
    """Whether `mlp` has the LlamaMLP form the fused gate/up kernel computes."""
    parts = [getattr(mlp, n, None) for n in ("gate_proj", "up_proj", "down_proj")]
    return (all(isinstance(p, nn.Linear) for p in parts)
            and _is_silu(getattr(mlp, "act_fn", None))
            and parts[0].bias is None and parts[1].bias is None)


class Int8RMSNormQuant(nn.Module):
    """Drop-in for a decoder layer's `input_layernorm` / `post_attention_layernorm` (LlamaRMSNorm,
    modeling_llama.py:53-67) in the W8A8 mode: the norm and the per-token quantization its W8A8
    consumers would each repeat run as one kernel, and the result travels as `QuantizedRows`.
    The bf16 weight stays a Parameter (the runner reads `model.dtype` off the first one)."""

    def __init__(self, norm: nn.Module) -> None:
        super().__init__()
        self.weight = norm.weight
        self.variance_epsilon = norm.variance_epsilon

    def forward(self, x: torch.Tensor) -> QuantizedRows:
        xq, sx, _ = ops.rmsnorm_quantize(x, self.weight, self.variance_epsilon)
        return QuantizedRows(xq, sx, x.shape, x.dtype)

    def extra_repr(self) -> str:
        return f"{tuple(self.weight.shape)}, eps={self.variance_epsilon}, quantize=per-token int8"


class PackedBf16Linear(nn.Module):
    """Drop-in for the bf16 `lm_head` (`nn.Linear(K, N, bias=False)`) the int8 path keeps in
    bf16: the reference calls it as `get_output_embeddings()(hidden)` (model_runner.py:306-307,
    decode_graph.py:140), which this module's `forward(x) -> y` serves. The weight is held in the
    packed bf16 tile layout (`ops.pack_bf16_weight`, buffer `wp`, the same bytes as the bf16
    matrix) and the product runs as `lse_bf16_decode_gemm`: the decode kernel up to 16 rows and
    bf16 tiles of the tiled kernel above. `unpacked_weight()` returns the row-major matrix."""

    def __init__(self, in_features: int, out_features: int,
                 device: torch.device | str | None = None) -> None:
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.register_buffer(
            "wp",
            torch.zeros(ops.packed_bf16_shape(out_features, in_features), dtype=torch.bfloat16,
                        device=device),
        )

    @classmethod
    def from_linear(cls, linear: nn.Linear) -> PackedBf16Linear:
        """Packs `linear.weight` (bf16, on the GPU, no bias) on its own device."""
        w = linear.weight.detach()
        if linear.bias is not None:
            raise RuntimeError("the packed bf16 linear has no bias term")
        if w.dtype != torch.bfloat16:
            raise RuntimeError(f"the packed bf16 linear needs a bf16 weight, got {w.dtype}")
        if w.device.type != "cuda":
            raise RuntimeError(f"the packed bf16 linear needs a CUDA (HIP) device, got {w.device}")
        k_align = _lib.query(_lib.Q_K_ALIGN)
        if linear.in_features % k_align:
            raise RuntimeError(f"the packed bf16 linear needs in_features % {k_align} == 0, got "
                               f"{linear.in_features}")
        mod = cls(linear.in_features, linear.out_features, w.device)
        mod.wp.copy_(ops.pack_bf16_weight(w))
        return mod

    def unpacked_weight(self) -> torch.Tensor:
        """The bf16 weight as a row-major (N, K) matrix."""
        return ops.unpack_bf16_weight(self.wp, self.out_features, self.in_features)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return ops.bf16_decode_linear(x, self.wp, self.out_features)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, packed bf16"
