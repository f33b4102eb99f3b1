"""MI355X (gfx950) int8 quantized Linear forward for llm-serving-engine.

The package directory name is not a Python identifier; `__graft_entry__.load_package()` imports
it as `llm_serving_engine_amd`.
"""

from . import ops
from ._lib import LIB_PATH, library
from .checkpoint import load_int8_checkpoint, save_int8_checkpoint
from .config import ModelConfig
from .int8_linear import (
    Int8GateUp,
    Int8GluMLP,
    Int8Linear,
    Int8RMSNormQuant,
    PackedBf16Linear,
    QuantizedRows,
    check_linear_supported,
)
from .quantize import check_int8_support, quantize_model_

__all__ = [
    "LIB_PATH",
    "Int8GateUp",
    "Int8GluMLP",
    "Int8Linear",
    "Int8RMSNormQuant",
    "ModelConfig",
    "PackedBf16Linear",
    "QuantizedRows",
    "check_int8_support",
    "check_linear_supported",
    "library",
    "load_int8_checkpoint",
    "ops",
    "quantize_model_",
    "save_int8_checkpoint",
]
