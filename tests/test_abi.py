"""The C ABI without a GPU: the library loads, exports every function include/lse_int8.h declares,
and rejects bad arguments with the documented status before any HIP call is made."""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

REPO_ROOT = Path(__file__).resolve().parent.parent
HEADERS = sorted((REPO_ROOT / "include").glob("*.h"))


def _declared_functions() -> set[str]:
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"^\s*[\w\s\*]*?\b(lse_\w+)\s*\(", text, flags=re.M))
    return names


def test_header_declares_the_entry_points():
    names = _declared_functions()
    assert {
        "lse_quantize_weight_per_channel", "lse_packed_weight_bytes", "lse_pack_weight",
        "lse_w8a16_gemm", "lse_w8a16_gemm_algo", "lse_workspace_bytes",
        "lse_quantize_act_per_token", "lse_w8a8_gemm", "lse_query", "lse_status_string",
    } <= names


def test_library_exports_every_declared_symbol(pkg):
    lib = pkg.library()
    exported = subprocess.run(
        ["nm", "-D", "--defined-only", str(pkg.LIB_PATH)], capture_output=True, text=True, check=True
    ).stdout
    for name in _declared_functions():
        assert re.search(rf"\bT {name}$", exported, flags=re.M), name
        assert getattr(lib, name) is not None


def test_binding_covers_the_header(pkg):
    from llm_serving_engine_amd import _lib

    assert set(_lib.SIGNATURES) == _declared_functions()


def test_query_values(pkg):
    from llm_serving_engine_amd import _lib

    assert _lib.query(_lib.Q_ABI_VERSION) == _lib.ABI_VERSION
    assert _lib.query(_lib.Q_K_ALIGN) == 16
    assert _lib.query(_lib.Q_DECODE_MAX_M) == 64
    assert 127 * 127 * _lib.query(_lib.Q_MAX_K) < 2**31
    assert _lib.query(_lib.Q_GFX_ARCH) == 950
    assert _lib.query(_lib.Q_NOALLOC_SCRATCH) == 32 << 20
    assert _lib.query(99) == -1


# A fake, 256-byte-aligned device address: every call below is rejected before it is used.
FAKE = ctypes.c_void_p(1 << 20)
E_NULL, E_SHAPE, E_ALIGN, E_RANGE, E_ALGO, E_WORKSPACE = -1, -2, -3, -4, -5, -6


@pytest.mark.parametrize(
    "args,status",
    [
        # (x, ldx, qp, s, y, ldy, M, N, K, algo)
        ((FAKE, 64, FAKE, FAKE, FAKE, 64, 1, 64, 60, 0), E_ALIGN),  # K % 16
        ((FAKE, 64, FAKE, FAKE, FAKE, 64, -1, 64, 64, 0), E_SHAPE),
        ((FAKE, 64, None, FAKE, FAKE, 64, 1, 64, 64, 0), E_NULL),
        ((FAKE, 64, FAKE, None, FAKE, 64, 1, 64, 64, 0), E_NULL),
        ((FAKE, 64, FAKE, FAKE, None, 64, 1, 64, 64, 0), E_NULL),
        ((None, 64, FAKE, FAKE, FAKE, 64, 1, 64, 64, 0), E_NULL),
        ((FAKE, 60, FAKE, FAKE, FAKE, 64, 2, 64, 64, 0), E_SHAPE),  # ldx < K
        ((FAKE, 68, FAKE, FAKE, FAKE, 64, 2, 64, 64, 0), E_ALIGN),  # ldx % 8
        ((FAKE, 64, FAKE, FAKE, ctypes.c_void_p((1 << 20) + 1), 64, 2, 64, 64, 0),
         E_ALIGN),
        ((FAKE, 64, FAKE, FAKE, FAKE, 32, 2, 64, 64, 0), E_SHAPE),  # ldy < N
        ((ctypes.c_void_p((1 << 20) + 8), 64, FAKE, FAKE, FAKE, 64, 1, 64, 64, 0),
         E_ALIGN),
        ((FAKE, 64, ctypes.c_void_p((1 << 20) + 4), FAKE, FAKE, 64, 1, 64, 64, 0),
         E_ALIGN),
        ((FAKE, 64, FAKE, FAKE, FAKE, 64, 65, 64, 64, 1), E_ALGO),  # decode M <= 64
        ((FAKE, 64, FAKE, FAKE, FAKE, 64, 1, 64, 64, 7), E_ALGO),
        ((FAKE, 1 << 20, FAKE, FAKE, FAKE, 64, 1, 64, 200_000, 0), E_RANGE),
        ((FAKE, 4096, FAKE, FAKE, FAKE, 1 << 20, 1, 1 << 20, 4096, 0), E_RANGE),
        ((FAKE, 1 << 23, FAKE, FAKE, FAKE, 64, 100, 64, 64, 2), E_RANGE),  # tiled x extent
    ],
)
def test_w8a16_rejects_bad_arguments(pkg, args, status):
    lib = pkg.library()
    assert lib.lse_w8a16_gemm_algo(*args, None, 0, None) == status
    assert lib.lse_status_string(status)


def test_workspace_query_and_rejections(pkg):
    lib = pkg.library()
    assert lib.lse_workspace_bytes(0, -1, 64, 64) == -1
    assert lib.lse_workspace_bytes(2, 1, 64, 64) == -1
    assert lib.lse_workspace_bytes(0, 257, 4096, 4096) == 0  # above 256 tokens none
    assert lib.lse_workspace_bytes(1, 0, 4096, 4096) == 0
    # 65..256 tokens over a narrow weight: the tiled kernel's K ranges, a class-wide count.
    assert lib.lse_workspace_bytes(0, 65, 4096, 14336) > 0
    for m in (65, 100, 128):
        assert lib.lse_workspace_bytes(0, m, 4096, 14336) * 65 == \
            lib.lse_workspace_bytes(0, 65, 4096, 14336) * m
    # 257..1024 tokens over a deep, narrow weight: 4 ranges up to 512 tokens, then 2 (W8A16).
    for m in (257, 400, 512):
        assert lib.lse_workspace_bytes(0, m, 4096, 14336) == 4 * m * 4096 * 4
        assert lib.lse_workspace_bytes(1, m, 4096, 14336) == 4 * m * 4096 * 4
    for m in (513, 1024):
        assert lib.lse_workspace_bytes(0, m, 4096, 14336) == 2 * m * 4096 * 4
        assert lib.lse_workspace_bytes(1, m, 4096, 14336) == 0
    assert lib.lse_workspace_bytes(0, 1025, 4096, 14336) == 0
    for mode in (0, 1):
        for m in (1, 16, 17, 33, 64, 65, 128, 129, 256, 257, 512, 1024):
            nbytes = lib.lse_workspace_bytes(mode, m, 4096, 14336)
            assert 0 <= nbytes <= 64 * m * (4096 + 15) and nbytes % 16 == 0
    args = (FAKE, 64, FAKE, FAKE, FAKE, 64, 2, 64, 64, 1)
    assert lib.lse_w8a16_gemm_algo(*args, FAKE, -1, None) == E_WORKSPACE
    assert lib.lse_w8a16_gemm_algo(*args, ctypes.c_void_p((1 << 20) + 8), 64, None) == E_WORKSPACE
    assert lib.lse_w8a8_gemm(FAKE, FAKE, FAKE, FAKE, FAKE, 64, None, 2, 64, 64, FAKE, -1,
                             None) == E_WORKSPACE


def test_empty_shapes_are_no_ops(pkg):
    lib = pkg.library()
    assert lib.lse_w8a16_gemm(None, 0, None, None, None, 0, 0, 0, 0, None, 0, None) == 0
    assert lib.lse_w8a16_gemm(None, 16, FAKE, FAKE, None, 0, 0, 64, 16, None, 0, None) == 0
    assert lib.lse_w8a8_gemm(None, None, FAKE, FAKE, None, 0, None, 0, 64, 16, None, 0, None) == 0
    assert lib.lse_quantize_act_per_token(None, 0, None, FAKE, 0, 16, None) == 0
    assert lib.lse_quantize_weight_per_channel(None, 0, None, FAKE, 0, 16, None) == 0
    assert lib.lse_pack_weight(None, 0, 16, None, None) == 0


def test_packed_sizes_and_pack_rejections(pkg):
    lib = pkg.library()
    assert lib.lse_packed_weight_bytes(4096, 4096) == 256 * 64 * 1024
    assert lib.lse_packed_weight_bytes(17, 80) == 2 * 2 * 1024
    assert lib.lse_packed_weight_bytes(-1, 16) == -1
    assert lib.lse_pack_weight(FAKE, 16, 40, FAKE, None) == E_ALIGN
    assert lib.lse_pack_weight(None, 16, 32, FAKE, None) == E_NULL
    assert lib.lse_pack_weight(FAKE, 16, 32, ctypes.c_void_p((1 << 20) + 8), None) == E_ALIGN
    assert lib.lse_pack_weight(FAKE, 1 << 20, 4096, FAKE, None) == E_RANGE


def test_quantizers_and_w8a8_reject_bad_arguments(pkg):
    lib = pkg.library()
    assert lib.lse_quantize_weight_per_channel(FAKE, 64, FAKE, FAKE, 4, 40, None) == E_ALIGN
    assert lib.lse_quantize_weight_per_channel(FAKE, 30, FAKE, FAKE, 4, 32, None) == E_SHAPE
    assert lib.lse_quantize_weight_per_channel(FAKE, 34, FAKE, FAKE, 4, 32, None) == E_ALIGN
    assert lib.lse_quantize_weight_per_channel(FAKE, 32, FAKE, None, 4, 32, None) == E_NULL
    assert lib.lse_quantize_act_per_token(FAKE, 32, FAKE, FAKE, -1, 32, None) == E_SHAPE
    assert lib.lse_quantize_act_per_token(FAKE, 36, FAKE, FAKE, 2, 32, None) == E_ALIGN
    assert lib.lse_quantize_act_per_token(None, 32, FAKE, FAKE, 2, 32, None) == E_NULL
    assert lib.lse_w8a8_gemm(FAKE, None, FAKE, FAKE, FAKE, 64, None, 2, 64, 64, None, 0, None) == E_NULL
    assert lib.lse_w8a8_gemm(FAKE, FAKE, FAKE, FAKE, FAKE, 64, None, 2, 64, 200_000, None, 0, None) == E_RANGE
    assert lib.lse_w8a8_gemm(FAKE, FAKE, FAKE, FAKE, FAKE, 64, ctypes.c_void_p((1 << 20) + 4),
                             2, 64, 64, None, 0, None) == E_ALIGN
    assert lib.lse_w8a8_gemm(None, FAKE, FAKE, FAKE, FAKE, 64, None, 2, 64, 64, None, 0, None) == E_NULL


def test_fused_w8a8_linear_eligibility_and_rejections(pkg):
    """The one-launch W8A8 path runs for small decode batches whose int8 rows fit the staged
    image (M <= 16, M * K <= 128 KB) and refuses everything else before any launch."""
    lib = pkg.library()
    assert lib.lse_w8a8_linear_supported(1, 4096) == 1
    assert lib.lse_w8a8_linear_supported(16, 8192) == 1
    assert lib.lse_w8a8_linear_supported(9, 14336) == 1   # 9 x 14336 bytes <= 128 KB
    assert lib.lse_w8a8_linear_supported(10, 14336) == 0
    assert lib.lse_w8a8_linear_supported(17, 4096) == 0
    assert lib.lse_w8a8_linear_supported(0, 4096) == 0
    assert lib.lse_w8a8_linear_supported(1, 40) == 0      # K not a multiple of 16
    assert lib.lse_w8a8_linear(FAKE, 64, FAKE, FAKE, FAKE, 64, None, 17, 64, 64, None) == E_ALGO
    assert lib.lse_w8a8_linear(FAKE, 64, FAKE, FAKE, FAKE, 64, None, -1, 64, 64, None) == E_SHAPE
    assert lib.lse_w8a8_linear(FAKE, 64, None, FAKE, FAKE, 64, None, 2, 64, 64, None) == E_NULL
    assert lib.lse_w8a8_linear(FAKE, 60, FAKE, FAKE, FAKE, 64, None, 2, 64, 64, None) == E_SHAPE
    assert lib.lse_w8a8_linear(FAKE, 64, FAKE, FAKE, FAKE, 64, ctypes.c_void_p((1 << 20) + 4),
                               2, 64, 64, None) == E_ALIGN
    assert lib.lse_w8a8_linear(None, 0, FAKE, FAKE, None, 0, None, 0, 64, 64, None) == 0


def test_status_strings(pkg):
    lib = pkg.library()
    for st in (0, E_NULL, E_SHAPE, E_ALIGN, E_RANGE, E_ALGO, E_WORKSPACE, -99):
        assert isinstance(lib.lse_status_string(st), bytes)


def test_glu_entry_points_reject_bad_arguments(pkg):
    lib = pkg.library()
    assert lib.lse_packed_glu_bytes(14336, 4096) == 2 * 896 * 64 * 1024
    assert lib.lse_packed_glu_bytes(20, 80) == 2 * 2 * 2 * 1024
    assert lib.lse_packed_glu_bytes(-1, 16) == -1
    assert lib.lse_pack_glu(FAKE, 16, 40, FAKE, None) == E_ALIGN
    assert lib.lse_pack_glu(FAKE, -1, 32, FAKE, None) == E_SHAPE
    assert lib.lse_pack_glu(None, 16, 32, FAKE, None) == E_NULL
    assert lib.lse_pack_glu(FAKE, 1 << 19, 4096, FAKE, None) == E_RANGE
    assert lib.lse_pack_glu(None, 0, 32, None, None) == 0
    # (x, ldx, qp, s, h, ldh, M, I, K, algo)
    ok = (FAKE, 64, FAKE, FAKE, FAKE, 64, 2, 64, 64, 0)
    cases = [
        ((FAKE, 64, FAKE, FAKE, FAKE, 64, 2, 64, 40, 0), E_ALIGN),
        ((FAKE, 64, FAKE, FAKE, FAKE, 64, 2, -1, 64, 0), E_SHAPE),
        ((FAKE, 64, FAKE, FAKE, FAKE, 32, 2, 64, 64, 0), E_SHAPE),  # ldh < I
        ((FAKE, 64, None, FAKE, FAKE, 64, 2, 64, 64, 0), E_NULL),
        ((FAKE, 64, FAKE, None, FAKE, 64, 2, 64, 64, 0), E_NULL),
        ((None, 64, FAKE, FAKE, FAKE, 64, 2, 64, 64, 0), E_NULL),
        ((FAKE, 64, FAKE, FAKE, FAKE, 64, 65, 64, 64, 1), E_ALGO),
        ((FAKE, 64, FAKE, FAKE, FAKE, 64, 2, 64, 64, 3), E_ALGO),
        ((FAKE, 64, FAKE, FAKE, FAKE, 64, 2, 64, 200_000, 0), E_RANGE),
        ((FAKE, 4096, FAKE, FAKE, FAKE, 1 << 19, 1, 1 << 19, 4096, 0), E_RANGE),
        ((FAKE, 1 << 23, FAKE, FAKE, FAKE, 64, 100, 64, 64, 2), E_RANGE),
    ]
    for args, status in cases:
        assert lib.lse_w8a16_glu(*args, None) == status, args
    assert lib.lse_w8a16_glu(*ok[:6], 0, 64, 64, 0, None) == 0  # M = 0
    # (xq, sx, qp, s, h, ldh, M, I, K)
    assert lib.lse_w8a8_glu(FAKE, None, FAKE, FAKE, FAKE, 64, 2, 64, 64, None) == E_NULL
    assert lib.lse_w8a8_glu(None, FAKE, FAKE, FAKE, FAKE, 64, 2, 64, 64, None) == E_NULL
    assert lib.lse_w8a8_glu(FAKE, FAKE, FAKE, FAKE, FAKE, 64, 2, 64, 200_000, None) == E_RANGE
    assert lib.lse_w8a8_glu(ctypes.c_void_p((1 << 20) + 4), FAKE, FAKE, FAKE, FAKE, 64, 2, 64,
                            64, None) == E_ALIGN
    assert lib.lse_w8a8_glu(FAKE, FAKE, FAKE, FAKE, FAKE, 16, 2, 64, 64, None) == E_SHAPE


def test_rmsnorm_quantize_rejects_bad_arguments(pkg):
    lib = pkg.library()
    # (x, ldx, weight, eps, xq, sx, normed, M, K)
    assert lib.lse_rmsnorm_quantize(FAKE, 64, FAKE, 1e-5, FAKE, FAKE, None, 2, 40, None) == E_ALIGN
    assert lib.lse_rmsnorm_quantize(FAKE, 64, None, 1e-5, FAKE, FAKE, None, 2, 64, None) == E_NULL
    assert lib.lse_rmsnorm_quantize(FAKE, 32, FAKE, 1e-5, FAKE, FAKE, None, 2, 64, None) == E_SHAPE
    assert lib.lse_rmsnorm_quantize(FAKE, 64, FAKE, -1.0, FAKE, FAKE, None, 2, 64, None) == E_SHAPE
    assert lib.lse_rmsnorm_quantize(FAKE, 64, ctypes.c_void_p((1 << 20) + 2), 1e-5, FAKE, FAKE,
                                    None, 2, 64, None) == E_ALIGN
    assert lib.lse_rmsnorm_quantize(None, 64, None, 1e-5, None, None, None, 0, 64, None) == 0
