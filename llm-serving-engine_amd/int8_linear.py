"""`Int8Linear`: the drop-in for `nn.Linear(K, N, bias=False)` on the engine's model path.

The reference calls its projections as plain modules, `attn.q_proj(normed)` and the like
(src/llm_serving_engine/model/model_runner.py:322-324, 369, 418; transformers
modeling_llama.py:175), so the replacement keeps exactly `forward(x) -> y` with x (..., K) and
y (..., N) in bf16 on the same device and the current stream. Quantized weights and scales are
buffers, not Parameters: the runner reads `model.dtype` off the first parameter
(model_runner.py:86,112) and must keep seeing bf16.

`qweight` holds the int8 weight in the packed tile layout the kernels stream (ops.pack_weight),
shape (ceil(N/16), ceil(K/64), 1024); `unpacked_qweight()` returns the row-major (N, K) matrix.
"""

from __future__ import annotations

import torch
from torch import nn

from . import _lib, ops

MODES = ("int8", "w8a8")


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

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.mode == "int8":
            y = ops.w8a16_linear(x, self.qweight, self.scales)
        else:
            y = ops.w8a8_linear(x, self.qweight, self.scales)
        return y if self.bias is None else y + self.bias

    def extra_repr(self) -> str:
        return (
            f"in_features={self.in_features}, out_features={self.out_features}, "
            f"mode={self.mode}, bias={self.bias is not None}"
        )


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
