"""W8A8 parity on the GPU: int32 accumulators bit-exact, the (acc * sx) * s epilogue bit-exact,
for the decode (M <= 64) and tiled (M > 64) kernels, against the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bf16_bits, to_bf16_tensor
from oracle import numerics as ora

pytestmark = pytest.mark.gpu

LLAMA_SHAPES = [(4096, 6144), (4096, 4096), (4096, 28672), (14336, 4096)]  # (K, N)


def _w8a8(pkg, dev, x_bits, q, s):
    x = to_bf16_tensor(x_bits, dev)
    xq, sx = pkg.ops.quantize_act_per_token(x)
    qp = pkg.ops.pack_weight(torch.from_numpy(q).to(dev))
    y, acc = pkg.ops.w8a8_gemm(xq, sx, qp, torch.from_numpy(s).to(dev), True)
    torch.cuda.synchronize()
    return xq.cpu().numpy(), sx.cpu().numpy(), acc.cpu().numpy(), bf16_bits(y)


def _check(pkg, dev, m, n, k, seed):
    x_bits, w = ora.seeded_inputs(seed, m, n, k, outliers=True)
    q, s = ora.quantize_weight_per_channel(w)
    xq, sx, acc, y = _w8a8(pkg, dev, x_bits, q, s)
    xq_ref, sx_ref = ora.quantize_act_per_token(x_bits)
    np.testing.assert_array_equal(xq, xq_ref)
    np.testing.assert_array_equal(sx, sx_ref)
    acc_ref = ora.w8a8_accumulate(xq_ref, q)
    np.testing.assert_array_equal(acc, acc_ref, err_msg=f"acc M={m} N={n} K={k}")
    np.testing.assert_array_equal(y, ora.w8a8_epilogue(acc_ref, sx_ref, s), err_msg=f"y M={m}")


@pytest.mark.parametrize("m", [1, 2, 16, 17, 32, 33, 64])
def test_decode_kernel_bit_exact(pkg, dev, m):
    _check(pkg, dev, m, 208, 1024, 500 + m)


@pytest.mark.parametrize("m", [1, 16, 17, 32, 33, 64])
@pytest.mark.parametrize("n,k", [(48, 4096), (4096, 128), (144, 3136), (16, 14336), (1000, 8208)])
def test_decode_split_panels_bit_exact(pkg, dev, m, n, k):
    """Few panels with a long K and many panels with a short K, staged and streamed
    activations, and (past 16 tokens) K split over four partial sums added in a second pass:
    the int32 sums stay exact."""
    _check(pkg, dev, m, n, k, 7 * m + n + k)


@pytest.mark.parametrize("m", [65, 128, 200, 512])
@pytest.mark.parametrize("n,k", [(128, 128), (100, 176), (256, 2048)])
def test_tiled_kernel_bit_exact(pkg, dev, m, n, k):
    _check(pkg, dev, m, n, k, m + n + k)


@pytest.mark.parametrize("m", [65, 129, 256])
@pytest.mark.parametrize("n,k", [(256, 14336), (272, 4096 + 48)])
def test_tiled_split_k_bit_exact(pkg, dev, m, n, k):
    """65..256 tokens over a narrow weight: K split into 8 ranges whose int32 partial sums a
    second pass adds, with a ragged last row tile and a 2-step last range ending in a K tail
    for (272, 4144). int32 sums are exact, so acc and y equal the oracle's bit for bit."""
    _check(pkg, dev, m, n, k, 3 * m + n + k)


@pytest.mark.parametrize("m", [257, 512, 513])
def test_tiled_deep_split_k_bit_exact(pkg, dev, m):
    """257..512 tokens over a deep, narrow weight: 4 K ranges of 256 x 128 int8 tiles (513 and
    up: no split in W8A8), bit for bit the oracle's accumulators and outputs."""
    nbytes = pkg.library().lse_workspace_bytes(1, m, 256, 14336)
    assert nbytes == (4 * m * 256 * 4 if m <= 512 else 0)
    _check(pkg, dev, m, 256, 14336, 11 * m + 3)


@pytest.mark.parametrize("n,k", [(1, 16), (17, 48), (45, 1072)])
def test_ragged_shapes_bit_exact(pkg, dev, n, k):
    for m in (1, 40, 90):
        _check(pkg, dev, m, n, k, 13 * n + k + m)


def test_extreme_operands_accumulate_exactly(pkg, dev):
    """All-±127 operands at K = 14336: |acc| = 127^2 K = 231,225,344 is the largest magnitude the
    Llama shapes reach, and it must land in int32 exactly."""
    k, n = 14336, 32
    xq = np.full((70, k), 127, np.int8)
    xq[1::2] = -127
    q = np.full((n, k), 127, np.int8)
    q[::3] = -127
    sx = np.ones(70, np.float32)
    s = np.ones(n, np.float32)
    qp = pkg.ops.pack_weight(torch.from_numpy(q).to(dev))
    for m in (5, 70):
        y, acc = pkg.ops.w8a8_gemm(
            torch.from_numpy(xq[:m].copy()).to(dev), torch.from_numpy(sx[:m].copy()).to(dev),
            qp, torch.from_numpy(s).to(dev), True,
        )
        torch.cuda.synchronize()
        np.testing.assert_array_equal(acc.cpu().numpy(), ora.w8a8_accumulate(xq[:m], q))


@pytest.mark.parametrize("k,n", LLAMA_SHAPES)
def test_llama_shapes_full_size(pkg, dev, k, n):
    """Config 3 at full size for M in {1, 32, 512}: accumulators checked exactly with an fp64
    GEMM on the GPU (integer products and sums below 2^53 are exact in fp64)."""
    torch.backends.cuda.matmul.allow_tf32 = False
    x_bits, w = ora.seeded_inputs(3000 + k + n, 512, n, k, outliers=True)
    q, s = pkg.ops.quantize_weight_per_channel(torch.from_numpy(w).to(dev))
    qp = pkg.ops.pack_weight(q)
    for m in (1, 32, 512):
        xq, sx = pkg.ops.quantize_act_per_token(to_bf16_tensor(x_bits[:m], dev))
        y, acc = pkg.ops.w8a8_gemm(xq, sx, qp, s, True)
        exact = (xq.double() @ q.double().t()).round().to(torch.int64)
        assert torch.equal(acc.to(torch.int64), exact), f"M={m} K={k} N={n}"
        y_ref = ora.w8a8_epilogue(acc.cpu().numpy(), sx.cpu().numpy(), s.cpu().numpy())
        np.testing.assert_array_equal(bf16_bits(y), y_ref)


@pytest.mark.parametrize("k,n", LLAMA_SHAPES)
def test_llama_shapes_at_4096_tokens(pkg, dev, k, n):
    """Config 3 at its largest size, M = 4096, every Llama-3-8B shape, with the outlier columns:
    the quantizer against the oracle, the accumulators exactly against an fp64 GEMM on the GPU
    (integer partial sums below 2^53 are exact in fp64, in any order), the epilogue against the
    oracle's, a block of rows at a time."""
    x_bits, w = ora.seeded_inputs(3500 + k + n, 4096, n, k, outliers=True)
    q, s = pkg.ops.quantize_weight_per_channel(torch.from_numpy(w).to(dev))
    del w
    qp = pkg.ops.pack_weight(q)
    xq, sx = pkg.ops.quantize_act_per_token(to_bf16_tensor(x_bits, dev))
    y, acc = pkg.ops.w8a8_gemm(xq, sx, qp, s, True)
    xq_ref, sx_ref = ora.quantize_act_per_token(x_bits)
    np.testing.assert_array_equal(xq.cpu().numpy(), xq_ref)
    np.testing.assert_array_equal(sx.cpu().numpy(), sx_ref)
    exact = (xq.double() @ q.double().t()).round().to(torch.int64)
    assert torch.equal(acc.to(torch.int64), exact), f"M=4096 K={k} N={n}"
    del exact
    s_host = s.cpu().numpy()
    for r0 in range(0, 4096, 1024):
        y_ref = ora.w8a8_epilogue(acc[r0:r0 + 1024].cpu().numpy(), sx_ref[r0:r0 + 1024], s_host)
        np.testing.assert_array_equal(bf16_bits(y[r0:r0 + 1024]), y_ref, err_msg=f"rows {r0}..")


@pytest.mark.parametrize("m,n", [(1500, 6000), (2048, 6144)])
def test_tiled_192_row_tiles_bit_exact(pkg, dev, m, n):
    """The shapes for which W8A16 takes 256 x 192 tiles (6000 and 6144 rows at 1500 and 2048
    tokens), in W8A8, which keeps the other tiles there: accumulators exactly against an fp64
    GEMM on the GPU, outputs against the oracle's epilogue."""
    k = 4096
    x_bits, w = ora.seeded_inputs(1930 + m + n, m, n, k, outliers=True)
    q, s = pkg.ops.quantize_weight_per_channel(torch.from_numpy(w).to(dev))
    del w
    qp = pkg.ops.pack_weight(q)
    xq, sx = pkg.ops.quantize_act_per_token(to_bf16_tensor(x_bits, dev))
    y, acc = pkg.ops.w8a8_gemm(xq, sx, qp, s, True)
    exact = (xq.double() @ q.double().t()).round().to(torch.int64)
    assert torch.equal(acc.to(torch.int64), exact), f"M={m} N={n}"
    del exact
    y_ref = ora.w8a8_epilogue(acc.cpu().numpy(), sx.cpu().numpy(), s.cpu().numpy())
    np.testing.assert_array_equal(bf16_bits(y), y_ref)


def test_acc_only_and_y_only(pkg, dev):
    x_bits, w = ora.seeded_inputs(61, 20, 64, 256, outliers=True)
    q, s = ora.quantize_weight_per_channel(w)
    xq, sx = pkg.ops.quantize_act_per_token(to_bf16_tensor(x_bits, dev))
    qt, st = pkg.ops.pack_weight(torch.from_numpy(q).to(dev)), torch.from_numpy(s).to(dev)
    y_only, none_acc = pkg.ops.w8a8_gemm(xq, sx, qt, st, want_acc=False, want_y=True)
    none_y, acc_only = pkg.ops.w8a8_gemm(xq, sx, qt, st, want_acc=True, want_y=False)
    assert none_acc is None and none_y is None
    y_both, acc_both = pkg.ops.w8a8_gemm(xq, sx, qt, st, want_acc=True, want_y=True)
    assert torch.equal(acc_only, acc_both) and torch.equal(y_only, y_both)


@pytest.mark.parametrize("m", [1, 2, 5, 16])
@pytest.mark.parametrize("n,k", [(272, 1024), (100, 176), (48, 4096), (33, 2064)])
def test_fused_linear_bit_exact(pkg, dev, m, n, k):
    """W8A8 from bf16 in one launch (the decode kernel quantizes while staging): xq and sx never
    leave the kernel, and acc and y equal the oracle's bit for bit, and the two-step path's."""
    assert pkg.library().lse_w8a8_linear_supported(m, k)
    x_bits, w = ora.seeded_inputs(900 + 7 * m + n + k, m, n, k, outliers=True)
    if m > 2:
        x_bits[2] = 0  # all-zero token: sx = 1, xq = 0
    q, s = ora.quantize_weight_per_channel(w)
    x = to_bf16_tensor(x_bits, dev)
    qp = pkg.ops.pack_weight(torch.from_numpy(q).to(dev))
    st = torch.from_numpy(s).to(dev)
    y, acc = pkg.ops.w8a8_linear(x, qp, st, want_acc=True, one_launch=True)
    torch.cuda.synchronize()
    xq_ref, sx_ref = ora.quantize_act_per_token(x_bits)
    acc_ref = ora.w8a8_accumulate(xq_ref, q)
    np.testing.assert_array_equal(acc.cpu().numpy(), acc_ref, err_msg=f"acc M={m} N={n} K={k}")
    np.testing.assert_array_equal(bf16_bits(y), ora.w8a8_epilogue(acc_ref, sx_ref, s))
    _, _, acc2, y2 = _w8a8(pkg, dev, x_bits, q, s)
    np.testing.assert_array_equal(acc.cpu().numpy(), acc2)
    np.testing.assert_array_equal(bf16_bits(y), y2)


def test_fused_linear_deep_k_and_strided_rows(pkg, dev):
    """The down projection's K (14336) at the largest M the staged image holds (9), and x rows
    with a stride past K."""
    m, n, k = 9, 64, 14336
    assert pkg.library().lse_w8a8_linear_supported(m, k)
    assert not pkg.library().lse_w8a8_linear_supported(m + 1, k)
    x_bits, w = ora.seeded_inputs(977, m, n, k, outliers=True)
    q, s = ora.quantize_weight_per_channel(w)
    wide = np.zeros((m, k + 64), np.uint16)
    wide[:, :k] = x_bits
    x = to_bf16_tensor(wide, dev)[:, :k]
    qp = pkg.ops.pack_weight(torch.from_numpy(q).to(dev))
    y, acc = pkg.ops.w8a8_linear(x, qp, torch.from_numpy(s).to(dev), want_acc=True,
                                 one_launch=True)
    torch.cuda.synchronize()
    xq_ref, sx_ref = ora.quantize_act_per_token(x_bits)
    acc_ref = ora.w8a8_accumulate(xq_ref, q)
    np.testing.assert_array_equal(acc.cpu().numpy(), acc_ref)
    np.testing.assert_array_equal(bf16_bits(y), ora.w8a8_epilogue(acc_ref, sx_ref, s))


@pytest.mark.parametrize("m", [20, 40])
def test_wide_weight_tiles_bit_exact(pkg, dev, m):
    """17..64 tokens over a weight of more than 1024 row tiles take 64 x 128 tiles of the tiled
    kernel: accumulators and outputs stay bit-exact, with a partial last tile and a K tail."""
    _check(pkg, dev, m, 16408, 80, 4100 + m)


@pytest.mark.parametrize("k,n", LLAMA_SHAPES)
def test_one_launch_route_at_llama_shapes(pkg, dev, k, n):
    """The one-launch W8A8 route (`lse_w8a8_linear`) at full Llama-3-8B size, for every M at
    which `w8a8_linear` takes it by default: 1, 2 and 3 rows at K = 4096 (o_proj and q/k/v at
    decode, model_runner.py:322-324,369) and 1 row at K = 14336 (down_proj,
    modeling_llama.py:175). The kernel keeps xq and sx to itself, so they are checked through
    what they determine: the quantizer of the two-step route equals the oracle's bit for bit,
    the one-launch accumulators equal the exact integer GEMM of the oracle's xq with q (fp64 on
    the GPU: integer sums below 2^53 are exact), and y equals the oracle's epilogue of those
    accumulators with the oracle's sx."""
    ms = [m for m in (1, 2, 3) if m * k <= pkg.ops.ONE_LAUNCH_W8A8_MAX_ELEMS]
    assert ms == ([1, 2, 3] if k == 4096 else [1])
    x_bits, w = ora.seeded_inputs(4400 + k + n, max(ms), n, k, outliers=True)
    x_bits[min(1, max(ms) - 1), :: 977] = 0  # a row with scattered zeros among the outliers
    q, s = pkg.ops.quantize_weight_per_channel(torch.from_numpy(w).to(dev))
    del w
    qp = pkg.ops.pack_weight(q)
    s_host = s.cpu().numpy()
    for m in ms:
        assert pkg.library().lse_w8a8_linear_supported(m, k)
        xm = x_bits[:m]
        xq_ref, sx_ref = ora.quantize_act_per_token(xm)
        xq2, sx2 = pkg.ops.quantize_act_per_token(to_bf16_tensor(xm, dev))
        np.testing.assert_array_equal(xq2.cpu().numpy(), xq_ref)
        np.testing.assert_array_equal(sx2.cpu().numpy(), sx_ref)
        y, acc = pkg.ops.w8a8_linear(to_bf16_tensor(xm, dev), qp, s, want_acc=True,
                                     one_launch=True)
        torch.cuda.synchronize()
        xq_t = torch.from_numpy(xq_ref).to(dev)
        exact = (xq_t.double() @ q.double().t()).round().to(torch.int64)
        assert torch.equal(acc.to(torch.int64), exact), f"one-launch acc M={m} K={k} N={n}"
        y_ref = ora.w8a8_epilogue(acc.cpu().numpy(), sx_ref, s_host)
        np.testing.assert_array_equal(bf16_bits(y), y_ref, err_msg=f"one-launch y M={m}")
        y2, acc2 = pkg.ops.w8a8_gemm(xq2, sx2, qp, s, True)
        assert torch.equal(acc, acc2) and torch.equal(y, y2), f"routes differ at M={m}"


@pytest.mark.parametrize("m,n,k", [(4096, 28672, 4096), (2048, 28672, 4096), (1500, 20000, 1024),
                                   (1500, 20004, 1024), (3000, 8200, 512)])
def test_staged_output_tiles_match_the_oracle(pkg, dev, m, n, k):
    """W8A8 launches of more than one round of 256 x 256 blocks without an int32 output write
    their bf16 tiles through LDS as whole row segments (gate_up at 4096 tokens: one launch of 7
    rounds; at 2048: the 3-round bulk launch); with the int32 output requested the kernels store
    directly. Both outputs bit-identical, and equal to the oracle's epilogue of the exact
    accumulators (checked against an fp64 GEMM on the GPU). Ragged M and N (partial edge tiles:
    1500 x 20000 and 3000 x 8200 in one launch of 474 and 396 blocks), and a row length not a
    multiple of 8 (20004), where the kernel keeps its direct stores."""
    x_bits, w = ora.seeded_inputs(7100 + m + n + k, m, n, k, outliers=True)
    q, s = pkg.ops.quantize_weight_per_channel(torch.from_numpy(w).to(dev))
    del w
    qp = pkg.ops.pack_weight(q)
    xq, sx = pkg.ops.quantize_act_per_token(to_bf16_tensor(x_bits, dev))
    y_staged, none_acc = pkg.ops.w8a8_gemm(xq, sx, qp, s, want_acc=False, want_y=True)
    y_direct, acc = pkg.ops.w8a8_gemm(xq, sx, qp, s, want_acc=True, want_y=True)
    assert none_acc is None
    assert torch.equal(y_staged, y_direct), f"M={m} N={n} K={k}"
    exact = (xq.double() @ q.double().t()).round().to(torch.int64)
    assert torch.equal(acc.to(torch.int64), exact), f"M={m} N={n} K={k}"
    del exact
    s_host, sx_host = s.cpu().numpy(), sx.cpu().numpy()
    for r0 in range(0, m, 1024):
        y_ref = ora.w8a8_epilogue(acc[r0:r0 + 1024].cpu().numpy(), sx_host[r0:r0 + 1024], s_host)
        np.testing.assert_array_equal(bf16_bits(y_staged[r0:r0 + 1024]), y_ref,
                                      err_msg=f"rows {r0}..")


@pytest.mark.parametrize("k", [64, 80, 1040])
def test_ping_pong_tile_with_odd_and_single_k_steps(pkg, dev, k):
    """The W8A8 256 x 256 tile runs its K loop in pairs of stages: one K step (64), two with a
    partial last one (80) and an odd count (1040: 17 steps) leave the last pair half or wholly
    empty. 1500 x 20000 takes that tile in one launch of 474 blocks (ragged in M and N), staged
    output without the int32 result, direct stores with it: accumulators exact against an fp64
    GEMM on the GPU, both outputs equal to the oracle's epilogue."""
    m, n = 1500, 20000
    x_bits, w = ora.seeded_inputs(7300 + k, m, n, k, outliers=True)
    q, s = pkg.ops.quantize_weight_per_channel(torch.from_numpy(w).to(dev))
    del w
    qp = pkg.ops.pack_weight(q)
    xq, sx = pkg.ops.quantize_act_per_token(to_bf16_tensor(x_bits, dev))
    y_staged, _ = pkg.ops.w8a8_gemm(xq, sx, qp, s, want_acc=False, want_y=True)
    y_direct, acc = pkg.ops.w8a8_gemm(xq, sx, qp, s, want_acc=True, want_y=True)
    exact = (xq.double() @ q.double().t()).round().to(torch.int64)
    assert torch.equal(acc.to(torch.int64), exact), f"K={k}"
    assert torch.equal(y_staged, y_direct), f"K={k}"
    y_ref = ora.w8a8_epilogue(acc.cpu().numpy(), sx.cpu().numpy(), s.cpu().numpy())
    np.testing.assert_array_equal(bf16_bits(y_direct), y_ref)
