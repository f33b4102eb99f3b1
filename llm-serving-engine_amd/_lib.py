"""ctypes binding of liblse_int8.so, the C ABI declared in include/lse_int8.h.

The library is built in-tree by build_ext.py. There is no fallback: if it is missing or fails to
load, every op raises RuntimeError, so a silent CPU or PyTorch path can never stand in for the
HIP kernels.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "liblse_int8.so"

# Every extern "C" symbol include/lse_int8.h declares, with (restype, argtypes).
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_INT = ctypes.c_int
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "lse_quantize_weight_per_channel": (_INT, [_P, _I64, _P, _P, _I64, _I64, _P]),
    "lse_packed_weight_bytes": (_I64, [_I64, _I64]),
    "lse_pack_weight": (_INT, [_P, _I64, _I64, _P, _P]),
    "lse_workspace_bytes": (_I64, [_INT, _I64, _I64, _I64]),
    "lse_w8a16_gemm": (_INT, [_P, _I64, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _I64, _P]),
    "lse_w8a16_gemm_noalloc": (_INT, [_P, _I64, _P, _P, _P, _I64, _I64, _I64, _I64, _P]),
    "lse_w8a16_gemm_algo": (
        _INT, [_P, _I64, _P, _P, _P, _I64, _I64, _I64, _I64, _INT, _P, _I64, _P]),
    "lse_quantize_act_per_token": (_INT, [_P, _I64, _P, _P, _I64, _I64, _P]),
    "lse_rmsnorm_quantize": (_INT, [_P, _I64, _P, ctypes.c_float, _P, _P, _P, _I64, _I64, _P]),
    "lse_w8a8_gemm": (_INT, [_P, _P, _P, _P, _P, _I64, _P, _I64, _I64, _I64, _P, _I64, _P]),
    "lse_w8a8_linear_supported": (_INT, [_I64, _I64]),
    "lse_w8a8_linear": (_INT, [_P, _I64, _P, _P, _P, _I64, _P, _I64, _I64, _I64, _P]),
    "lse_packed_glu_bytes": (_I64, [_I64, _I64]),
    "lse_pack_glu": (_INT, [_P, _I64, _I64, _P, _P]),
    "lse_w8a16_glu": (_INT, [_P, _I64, _P, _P, _P, _I64, _I64, _I64, _I64, _INT, _P]),
    "lse_w8a8_glu": (_INT, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P]),
    "lse_packed_bf16_weight_bytes": (_I64, [_I64, _I64]),
    "lse_pack_bf16_weight": (_INT, [_P, _I64, _I64, _I64, _P, _P]),
    "lse_bf16_decode_gemm": (_INT, [_P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P]),
    "lse_paged_attention_workspace_bytes": (_I64, [_I64] * 7),
    "lse_paged_attention": (_INT, [_P, _I64, _I64, _P, _P, _I64, _I64, _I64, _P, _I64, _P, _P, _P,
                                   _P, _P, _I64, _I64] + [_I64] * 7 + [ctypes.c_float, _P, _I64,
                                                                        _P]),
    "lse_query": (_I64, [_INT]),
    "lse_status_string": (ctypes.c_char_p, [_INT]),
}

# Mirrors of the header's enums.
LSE_OK = 0
ALGO_AUTO, ALGO_DECODE, ALGO_PREFILL = 0, 1, 2
MODE_W8A16, MODE_W8A8 = 0, 1
E_WORKSPACE, E_SCRATCH = -6, -7
Q_ABI_VERSION, Q_K_ALIGN, Q_DECODE_MAX_M, Q_MAX_K, Q_GFX_ARCH = 0, 1, 2, 3, 4
Q_NOALLOC_SCRATCH = 5
ABI_VERSION = 12

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def library() -> ctypes.CDLL:
    """The loaded library, with argtypes bound. Raises RuntimeError when it is not built."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH.name} is not built: run __graft_entry__.build() "
                "(or python llm-serving-engine_amd/build_ext.py) first"
            )
        try:
            lib = ctypes.CDLL(str(LIB_PATH))
        except OSError as e:
            raise RuntimeError(f"cannot load {LIB_PATH}: {e}") from e
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.lse_query(Q_ABI_VERSION)
        if version != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH.name} ABI {version}, this binding expects {ABI_VERSION}")
        _lib = lib
        return lib


def check(status: int, what: str) -> None:
    """Raises RuntimeError for a non-zero status, the error type the engine's GPU worker
    classifies (a rejected argument is negative, a HIP launch error positive)."""
    if status != LSE_OK:
        msg = library().lse_status_string(status).decode()
        raise RuntimeError(f"{what} failed with status {status}: {msg}")


def query(key: int) -> int:
    return int(library().lse_query(key))
