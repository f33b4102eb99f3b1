"""MI355X (gfx950) int8 quantized Linear forward for llm-serving-engine.

The package directory name is not a Python identifier; `__graft_entry__.load_package()` imports
it as `llm_serving_engine_amd`.
"""

from . import ops
from ._lib import LIB_PATH, library
from .config import ModelConfig
from .int8_linear import Int8GateUp, Int8GluMLP, Int8Linear, check_linear_supported
from .quantize import check_int8_support, quantize_model_

__all__ = [
    "LIB_PATH",
    "Int8GateUp",
    "Int8GluMLP",
    "Int8Linear",
    "ModelConfig",
    "check_int8_support",
    "check_linear_supported",
    "library",
    "ops",
    "quantize_model_",
]
