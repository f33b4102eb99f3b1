"""`ModelConfig` with the reference's int8 switch (src/llm_serving_engine/config.py:27-49).

Field names, defaults and env-var names follow the reference so a deployment's environment
carries over. `quantize` takes "none", "int8" (weight-only W8A16, the reference's meaning at
model_runner.py:45-46) or "w8a8" (dynamic per-token activations). The int8 kernels compute in
bf16, so `dtype` must be "bfloat16" whenever `quantize` is not "none".
"""

from __future__ import annotations

import os
from dataclasses import dataclass

QUANTIZE_MODES = ("none", "int8", "w8a8")


def _env_str(name: str, default: str) -> str:
    return os.environ.get(name, default)


def _env_bool(name: str, default: bool) -> bool:
    return os.environ.get(name, str(default)).lower() in ("1", "true", "yes")


@dataclass
class ModelConfig:
    model_name_or_path: str = "unsloth/Llama-3.2-3B-Instruct"
    device: str = "cuda"
    dtype: str = "float16"
    quantize: str = "none"  # "none", "int8" (W8A16) or "w8a8"
    use_custom_kernels: bool = True
    use_cuda_graphs: bool = True

    @classmethod
    def from_env(cls) -> ModelConfig:
        return cls(
            model_name_or_path=_env_str("LLM_MODEL", cls.model_name_or_path),
            device=_env_str("LLM_DEVICE", cls.device),
            dtype=_env_str("LLM_DTYPE", cls.dtype),
            quantize=_env_str("LLM_QUANTIZE", cls.quantize),
            use_custom_kernels=_env_bool("LLM_USE_CUSTOM_KERNELS", cls.use_custom_kernels),
            use_cuda_graphs=_env_bool("LLM_USE_CUDA_GRAPHS", cls.use_cuda_graphs),
        )

    def validate_quantize(self) -> None:
        """Raises for a switch value or dtype the int8 path cannot serve."""
        if self.quantize not in QUANTIZE_MODES:
            raise ValueError(f"quantize must be one of {QUANTIZE_MODES}, got {self.quantize!r}")
        if self.quantize != "none" and self.dtype != "bfloat16":
            raise RuntimeError(
                f"quantize={self.quantize!r} computes in bfloat16; set dtype='bfloat16' "
                f"(LLM_DTYPE), got {self.dtype!r}"
            )
