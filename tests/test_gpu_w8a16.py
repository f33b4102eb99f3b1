"""W8A16 parity on the GPU: both kernel families (decode M <= 64, prefill GEMM) against the
oracle on identical seeded inputs, through the C ABI.

Tolerance (north star: rel <= 1e-2 after fp32 accumulation): max-abs error <= 1e-2 * max|golden|
and elementwise relative error <= 1e-2 where |golden| > 1e-3 * max|golden|; golden in fp64.
Expected error is one bf16 rounding (2^-9) plus fp32 accumulation (~K * 2^-24).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bf16_bits, to_bf16_tensor
from oracle import numerics as ora

pytestmark = pytest.mark.gpu

DECODE, PREFILL = 1, 2
LLAMA_SHAPES = [(4096, 6144), (4096, 4096), (4096, 28672), (14336, 4096)]  # (K, N)


def _run(pkg, dev, x_bits, q, s, algo, ldy_pad=0):
    m, k = x_bits.shape
    n = q.shape[0]
    x = to_bf16_tensor(x_bits, dev)
    qt = pkg.ops.pack_weight(torch.from_numpy(q).to(dev))
    st = torch.from_numpy(s).to(dev)
    if ldy_pad:
        sentinel = torch.full((m, n + ldy_pad), -7.0, dtype=torch.bfloat16, device=dev)
        lib = pkg.library()
        ws = pkg.ops.workspace(0, m, n, k, dev)
        status = lib.lse_w8a16_gemm_algo(
            x.data_ptr(), k, qt.data_ptr(), st.data_ptr(), sentinel.data_ptr(), n + ldy_pad,
            m, n, k, algo, ws.data_ptr() if ws is not None else None,
            ws.numel() if ws is not None else 0, torch.cuda.current_stream().cuda_stream,
        )
        assert status == 0
        torch.cuda.synchronize()
        pad = sentinel[:, n:]
        assert torch.all(pad == -7.0), "kernel wrote outside y's rows"
        return bf16_bits(sentinel[:, :n])
    y = pkg.ops.w8a16_linear(x, qt, st, algo=algo)
    torch.cuda.synchronize()
    return bf16_bits(y)


def _check(pkg, dev, m, n, k, seed, algo):
    x_bits, w = ora.seeded_inputs(seed, m, n, k)
    q, s = ora.quantize_weight_per_channel(w)
    y = _run(pkg, dev, x_bits, q, s, algo)
    ok, msg = ora.within_tolerance(y, ora.w8a16_golden(x_bits, q, s))
    assert ok, f"M={m} N={n} K={k} algo={algo}: {msg}"
    return x_bits, q, s, y


def test_config0_gemv(pkg, dev):
    """Config 0: M=1, K=N=2048, seeded x ~ N(0,1) bf16, W ~ N(0, 0.02)."""
    _check(pkg, dev, 1, 2048, 2048, 0, DECODE)


def test_pack_weight_bit_exact(pkg, dev):
    """The GPU packer against the oracle's layout, with padding past N and K."""
    rng = np.random.default_rng(3)
    for n, k in ((1, 16), (37, 80), (272, 1024), (4096, 14336 + 48)):
        q = rng.integers(-127, 128, (n, k)).astype(np.int8)
        qp = pkg.ops.pack_weight(torch.from_numpy(q).to(dev))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(qp.cpu().numpy(), ora.pack_weight(q), err_msg=f"{n}x{k}")
        np.testing.assert_array_equal(pkg.ops.unpack_weight(qp, n, k).cpu().numpy(), q)


@pytest.mark.parametrize("m", [1, 2, 7, 8, 15, 16, 17, 31, 32, 33, 48, 63, 64])
def test_decode_all_m_tiles(pkg, dev, m):
    _check(pkg, dev, m, 272, 1024, 100 + m, DECODE)


@pytest.mark.parametrize("m", [1, 16, 17, 32, 33, 64])
@pytest.mark.parametrize(
    "n,k", [(48, 4096), (4096, 128), (144, 3136), (1000, 1040), (16, 14336), (1000, 8208)]
)
def test_decode_split_panels(pkg, dev, m, n, k):
    """Few panels with a long K, many panels with a short K, a K tail past the last whole unit,
    and activations both staged whole and streamed through the LDS ring. With more than 16
    tokens, (16, 14336) and (1000, 8208) split K and add partial sums in a second pass: the
    latter with a partial last panel, a shorter last K range and a 16-wide K tail."""
    _check(pkg, dev, m, n, k, 11 * m + n + k, DECODE)


def test_decode_rejects_a_short_workspace(pkg, dev):
    """A split-K shape needs a workspace; a smaller one is refused before any launch."""
    m, n, k = 40, 4096, 14336
    need = pkg.library().lse_workspace_bytes(0, m, n, k)
    assert need >= 4 * m * n * 4
    x = torch.zeros(m, k, dtype=torch.bfloat16, device=dev)
    qp = torch.zeros(pkg.ops.packed_shape(n, k), dtype=torch.int8, device=dev)
    s = torch.ones(n, dtype=torch.float32, device=dev)
    y = torch.full((m, n), 3.0, dtype=torch.bfloat16, device=dev)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    lib = pkg.library()
    args = (x.data_ptr(), k, qp.data_ptr(), s.data_ptr(), y.data_ptr(), n, m, n, k, DECODE)
    assert lib.lse_w8a16_gemm_algo(*args, ws.data_ptr(), need - 16, stream) == -6
    assert lib.lse_w8a16_gemm_algo(*args, None, 0, stream) == -6
    torch.cuda.synchronize()
    assert torch.all(y == 3.0)
    assert lib.lse_w8a16_gemm_algo(*args, ws.data_ptr(), need, stream) == 0
    torch.cuda.synchronize()
    assert torch.all(y == 0.0)


@pytest.mark.parametrize("m", [17, 32, 33, 64])
@pytest.mark.parametrize("n,k", [(1024, 4096), (768, 4096), (100, 2064), (1000, 4096 + 48)])
def test_decode_stationary_slice(pkg, dev, m, n, k):
    """17..64 tokens over at most 64 row tiles (k/v projections, tensor-parallel q/k/v shards):
    workgroups of four row tiles over one of up to 8 K ranges, the activation slice of the range
    staged once in LDS, partial sums added in a second pass. (100, 2064): 33 K steps in 7 ranges
    of 5 with a 3-step last range; (1000, 4144): a ragged last row tile and 65 K steps in 8 ranges
    of 9, the last ending in a 48-wide K tail."""
    _check(pkg, dev, m, n, k, 13 * m + n + k, DECODE)


@pytest.mark.parametrize(
    "n,k", [(1, 16), (15, 48), (16, 64), (17, 80), (100, 112), (33, 2064), (64, 4096 + 48),
            (16392, 80)]
)
def test_decode_ragged_shapes(pkg, dev, n, k):
    """N not a multiple of 16, K tails of 16/48 past the 64-wide superstep. (16392, 80): a weight
    wide enough (1025 row tiles) that 17..64 tokens take the 32 x 128 or 64 x 128 tiled route,
    with a partial last tile and a K tail."""
    for m in (1, 5, 20, 40):
        _check(pkg, dev, m, n, k, 7 * n + k, DECODE)


@pytest.mark.parametrize("m", [65, 100, 128, 129, 300])
@pytest.mark.parametrize("n,k", [(128, 64), (200, 112), (96, 1040), (384, 2048)])
def test_prefill_ragged_shapes(pkg, dev, m, n, k):
    _check(pkg, dev, m, n, k, 3 * m + n + k, PREFILL)


def test_prefill_small_m_matches_tolerance(pkg, dev):
    """The prefill kernel also accepts M <= 64 (one partly filled block)."""
    _check(pkg, dev, 5, 256, 512, 11, PREFILL)


@pytest.mark.parametrize("algo", [DECODE, PREFILL])
def test_unit_vector_selects_one_column(pkg, dev, algo):
    """x = e_k makes y[:, n] the single product bf16(fl32(q[n,k] * s[n])) exactly."""
    k, n = 256, 48
    _, w = ora.seeded_inputs(5, 1, n, k)
    q, s = ora.quantize_weight_per_channel(w)
    cols = [0, 17, 100, 255]
    x = np.zeros((len(cols), k), np.float32)
    for i, c in enumerate(cols):
        x[i, c] = 1.0
    y = _run(pkg, dev, ora.f32_to_bf16_bits(x), q, s, algo)
    expect = ora.f32_to_bf16_bits(q[:, cols].T.astype(np.float32) * s[None, :])
    np.testing.assert_array_equal(y, expect)


@pytest.mark.parametrize("algo", [DECODE, PREFILL])
def test_unit_scale_small_integers_are_exact(pkg, dev, algo):
    """With s = 1 and small integer x, every partial sum is an exact fp32 integer below 2^8·K,
    and the bf16 rounding of the total is the only rounding."""
    rng = np.random.default_rng(9)
    m, n, k = 9, 40, 512
    x = rng.integers(-3, 4, (m, k)).astype(np.float32)
    q = rng.integers(-127, 128, (n, k)).astype(np.int8)
    s = np.ones(n, np.float32)
    y = _run(pkg, dev, ora.f32_to_bf16_bits(x), q, s, algo)
    exact = x.astype(np.int64) @ q.astype(np.int64).T
    np.testing.assert_array_equal(y, ora.f32_to_bf16_bits(exact.astype(np.float32)))


@pytest.mark.parametrize("algo", [DECODE, PREFILL])
def test_output_stride_guard_band(pkg, dev, algo):
    """ldy > N: the columns between N and ldy keep their sentinel."""
    x_bits, w = ora.seeded_inputs(21, 70 if algo == PREFILL else 9, 52, 320)
    q, s = ora.quantize_weight_per_channel(w)
    y = _run(pkg, dev, x_bits, q, s, algo, ldy_pad=12)
    assert ora.within_tolerance(y, ora.w8a16_golden(x_bits, q, s))[0]


@pytest.mark.parametrize(
    "k,n", [(4096, 512), (14336, 4096), (1024, 6144), (8192, 6400), (256, 16400), (4096, 1024)])
def test_decode_rows_are_batch_invariant(pkg, dev, k, n):
    """A row's result does not depend on M or on the other rows within a token class (M <= 16,
    17..32, 33..64): the graphed decode runs a padded power-of-two bucket while eager decode runs
    the exact batch, and a bucket lies in the same class as the batch it pads, so both must agree
    bitwise. Across class boundaries rows agree to the tolerance."""
    x_bits, w = ora.seeded_inputs(31, 64, n, k)
    q, s = ora.quantize_weight_per_channel(w)
    top = {16: _run(pkg, dev, x_bits[:16], q, s, DECODE),
           32: _run(pkg, dev, x_bits[:32], q, s, DECODE),
           64: _run(pkg, dev, x_bits, q, s, DECODE)}
    for m, cls in ((1, 16), (3, 16), (8, 16), (15, 16), (17, 32), (31, 32), (33, 64), (63, 64)):
        part = _run(pkg, dev, x_bits[:m], q, s, DECODE)
        np.testing.assert_array_equal(part, top[cls][:m], err_msg=f"M={m}")
    for m, cls in ((40, 64), (5, 16), (20, 32)):
        padded = x_bits[:cls].copy()
        padded[m:] = 0
        np.testing.assert_array_equal(_run(pkg, dev, padded, q, s, DECODE)[:m], top[cls][:m])
    golden = ora.w8a16_golden(x_bits[:16], q, s)
    for cls in (16, 32, 64):
        assert ora.within_tolerance(top[cls][:16], golden)[0]


@pytest.mark.parametrize("k,n", [(1024, 256), (14336, 512)])
def test_prefill_rows_are_batch_invariant(pkg, dev, k, n):
    """The tiled route's token classes (65..128 and 129..256, which may split K over a narrow
    weight; 257..512 and 513..1024, which split K over a deep, narrow one; and above): inside a
    class a row's bits do not depend on M, on the other rows or on zero padding up to the
    class's largest M; across classes rows agree to the tolerance."""
    x_bits, w = ora.seeded_inputs(32, 1100, n, k)
    q, s = ora.quantize_weight_per_channel(w)
    top = {c: _run(pkg, dev, x_bits[:c], q, s, PREFILL) for c in (128, 256, 512, 1024, 1100)}
    for m, cls in ((65, 128), (100, 128), (127, 128), (129, 256), (200, 256), (255, 256),
                   (257, 512), (300, 512), (511, 512), (513, 1024), (700, 1024), (1025, 1100)):
        np.testing.assert_array_equal(_run(pkg, dev, x_bits[:m], q, s, PREFILL),
                                      top[cls][:m], err_msg=f"M={m}")
    for m, cls in ((70, 128), (150, 256), (400, 512), (600, 1024)):
        padded = x_bits[:cls].copy()
        padded[m:] = 0
        np.testing.assert_array_equal(_run(pkg, dev, padded, q, s, PREFILL)[:m], top[cls][:m])
    golden = ora.w8a16_golden(x_bits[:128], q, s)
    for cls in top:
        assert ora.within_tolerance(top[cls][:128], golden)[0]


@pytest.mark.parametrize("m", [257, 512, 513, 1024])
def test_prefill_deep_split_k(pkg, dev, m):
    """257..1024 tokens over a deep, narrow weight (at least 128 K steps): 4 K ranges at
    257..512 tokens, 2 at 513..1024, of 256 x 128 tiles, added by the second pass."""
    nbytes = pkg.library().lse_workspace_bytes(0, m, 512, 14336)
    assert nbytes == (4 if m <= 512 else 2) * m * 512 * 4
    _check(pkg, dev, m, 512, 14336, 7 * m + 1, PREFILL)


@pytest.mark.parametrize("m", [65, 100, 128, 129, 256])
@pytest.mark.parametrize("n,k", [(512, 14336), (272, 4096 + 48), (4096, 1024)])
def test_prefill_split_k(pkg, dev, m, n, k):
    """65..256 tokens over a narrow weight: the tiled kernel splits K into up to 8 ranges whose
    partial sums a second pass adds. (512, 14336): 8 ranges of 28 steps; (272, 4144): a ragged
    last row tile, 65 steps in ranges of 9 with a 2-step last range ending in a 48-wide K tail;
    (4096, 1024): 64 tiles of 64 x 128 and 2 ranges at 65..128 tokens."""
    _check(pkg, dev, m, n, k, 5 * m + n + k, PREFILL)


def test_prefill_rejects_a_short_workspace(pkg, dev):
    """A split tiled shape (down_proj at 100 tokens) needs a workspace; a smaller one is refused
    before any launch, and the decode-range bound covers either algorithm."""
    m, n, k = 100, 4096, 14336
    lib = pkg.library()
    need = lib.lse_workspace_bytes(0, m, n, k)
    assert need >= 2 * m * n * 4
    assert lib.lse_workspace_bytes(0, m, n, k) <= 64 * m * (n + 15)
    x = torch.zeros(m, k, dtype=torch.bfloat16, device=dev)
    qp = torch.zeros(pkg.ops.packed_shape(n, k), dtype=torch.int8, device=dev)
    s = torch.ones(n, dtype=torch.float32, device=dev)
    y = torch.full((m, n), 3.0, dtype=torch.bfloat16, device=dev)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    args = (x.data_ptr(), k, qp.data_ptr(), s.data_ptr(), y.data_ptr(), n, m, n, k, PREFILL)
    assert lib.lse_w8a16_gemm_algo(*args, ws.data_ptr(), need - 16, stream) == -6
    assert lib.lse_w8a16_gemm_algo(*args, None, 0, stream) == -6
    torch.cuda.synchronize()
    assert torch.all(y == 3.0)
    assert lib.lse_w8a16_gemm_algo(*args, ws.data_ptr(), need, stream) == 0
    torch.cuda.synchronize()
    assert torch.all(y == 0.0)


def test_repeat_calls_are_deterministic(pkg, dev):
    x_bits, w = ora.seeded_inputs(33, 64, 1024, 2048)
    q, s = ora.quantize_weight_per_channel(w)
    for algo in (DECODE, PREFILL):
        a = _run(pkg, dev, x_bits, q, s, algo)
        b = _run(pkg, dev, x_bits, q, s, algo)
        np.testing.assert_array_equal(a, b)


def _torch_fp32_reference(x, q, s):
    """Plain PyTorch fp32 reference of the same op on the GPU: dequantize, fp32 GEMM."""
    return (x.float() @ q.float().t()) * s[None, :]


@pytest.mark.parametrize("k,n", LLAMA_SHAPES)
def test_llama_decode_shapes_full_size(pkg, dev, k, n):
    """Config 1 at full size: M in {1, 8, 32, 64} against a torch fp32 reference on the GPU,
    and the weight quantizer against the oracle's digest-free invariants."""
    gen = torch.Generator(device="cpu").manual_seed(1000 + k + n)
    w = (torch.randn(n, k, generator=gen) * 0.02).to(dev)
    q, s = pkg.ops.quantize_weight_per_channel(w)
    qp = pkg.ops.pack_weight(q)
    for m in (1, 8, 32, 64):
        x = torch.randn(m, k, generator=gen).to(torch.bfloat16).to(dev)
        y = pkg.ops.w8a16_linear(x, qp, s, algo=DECODE)
        ref = _torch_fp32_reference(x, q, s).double().cpu().numpy()
        ok, msg = ora.within_tolerance(bf16_bits(y), ref)
        assert ok, f"M={m} K={k} N={n}: {msg}"


def check_rows_in_chunks(y, golden, rows=1024):
    """The oracle's W8A16 rule over blocks of `rows` rows (each against its own max|golden|, no
    looser than one check of the whole matrix): y bf16 and golden fp64 on the GPU, compared on
    the host a block at a time so a (8192, 28672) product never sits in host memory at once."""
    for r0 in range(0, y.shape[0], rows):
        ok, msg = ora.within_tolerance(bf16_bits(y[r0:r0 + rows]),
                                       golden[r0:r0 + rows].cpu().numpy())
        if not ok:
            return False, f"rows {r0}..{r0 + rows}: {msg}"
    return True, "ok"


@pytest.mark.parametrize("k,n", LLAMA_SHAPES)
def test_llama_prefill_shapes_at_8192_tokens(pkg, dev, k, n):
    """Config 2 at its largest size, M = 8192, every Llama-3-8B shape, against the fp64 product of
    the same bf16 activations and dequantized weights on the GPU."""
    gen = torch.Generator(device="cpu").manual_seed(2500 + k + n)
    w = (torch.randn(n, k, generator=gen) * 0.02).to(dev)
    q, s = pkg.ops.quantize_weight_per_channel(w)
    del w
    qp = pkg.ops.pack_weight(q)
    x = torch.randn(8192, k, generator=gen).to(torch.bfloat16).to(dev)
    y = pkg.ops.w8a16_linear(x, qp, s, algo=PREFILL)
    golden = (x.double() @ q.double().t()) * s.double()[None, :]
    ok, msg = check_rows_in_chunks(y, golden)
    assert ok, f"M=8192 K={k} N={n}: {msg}"


@pytest.mark.parametrize("k,n", LLAMA_SHAPES)
def test_llama_prefill_shapes_full_size(pkg, dev, k, n):
    """Config 2 at M = 65, 128, 129, 256 (K split over the narrow shapes), 512 and 2048 vs torch
    fp32 on the GPU (8192 in the test above)."""
    gen = torch.Generator(device="cpu").manual_seed(2000 + k + n)
    w = (torch.randn(n, k, generator=gen) * 0.02).to(dev)
    q, s = pkg.ops.quantize_weight_per_channel(w)
    qp = pkg.ops.pack_weight(q)
    for m in (65, 128, 129, 256, 512, 2048):
        x = torch.randn(m, k, generator=gen).to(torch.bfloat16).to(dev)
        y = pkg.ops.w8a16_linear(x, qp, s, algo=PREFILL)
        ref = _torch_fp32_reference(x, q, s).double().cpu().numpy()
        ok, msg = ora.within_tolerance(bf16_bits(y), ref)
        assert ok, f"M={m} K={k} N={n}: {msg}"


def test_prefill_96_row_tiles(pkg, dev):
    """65..96 tokens over a wide weight run in one block row of 96 x 128 tiles (N 17000: 133
    blocks, the last with 8 of its rows; K 1040: a 16-wide tail): against the oracle at 65 and 96
    tokens, and row for row the same bits as the same rows inside 100 tokens (128 x 128 tiles)."""
    n, k = 17000, 1040
    x_bits, w = ora.seeded_inputs(9600, 100, n, k)
    q, s = ora.quantize_weight_per_channel(w)
    x = to_bf16_tensor(x_bits, dev)
    qp = pkg.ops.pack_weight(torch.from_numpy(q).to(dev))
    st = torch.from_numpy(s).to(dev)
    y100 = bf16_bits(pkg.ops.w8a16_linear(x, qp, st, algo=PREFILL))
    for m in (65, 96):
        y = bf16_bits(pkg.ops.w8a16_linear(x[:m], qp, st, algo=PREFILL))
        ok, msg = ora.within_tolerance(y, ora.w8a16_golden(x_bits[:m], q, s))
        assert ok, f"M={m}: {msg}"
        np.testing.assert_array_equal(y, y100[:m])


@pytest.mark.parametrize("m,n", [(1500, 6000), (2048, 6144)])
def test_prefill_192_row_tiles(pkg, dev, m, n):
    """6000 and 6144 rows at 1500 and 2048 tokens: on 256 CUs the tile model picks 256 x 192
    tiles (one round of 192 or 256 blocks; 6000 ends in a block of 3 of its 12 row tiles), whose
    eight waves take 12 weight tiles in two loads each, the last four past the tiles. Against the
    fp64 product on the GPU, and row for row the same bits as the first 1100 rows run alone
    (128 x 128 tiles): every tile sums K in increasing order."""
    k = 4096
    gen = torch.Generator(device="cpu").manual_seed(1920 + m + n)
    w = (torch.randn(n, k, generator=gen) * 0.02).to(dev)
    q, s = pkg.ops.quantize_weight_per_channel(w)
    del w
    qp = pkg.ops.pack_weight(q)
    x = torch.randn(m, k, generator=gen).to(torch.bfloat16).to(dev)
    y = pkg.ops.w8a16_linear(x, qp, s, algo=PREFILL)
    golden = (x.double() @ q.double().t()) * s.double()[None, :]
    ok, msg = check_rows_in_chunks(y, golden)
    assert ok, f"M={m} N={n}: {msg}"
    del golden
    y_small = pkg.ops.w8a16_linear(x[:1100], qp, s, algo=PREFILL)
    assert torch.equal(y[:1100].view(torch.int16), y_small.view(torch.int16))


@pytest.mark.parametrize("mode,n,m", [
    ("w8a16", 28672, 2048), ("w8a8", 28672, 2048), ("glu", 28672, 2048),
    ("w8a16", 6144, 4096), ("w8a8", 6144, 4096)])
def test_tail_split_launch_changes_no_bit(pkg, dev, mode, n, m):
    """gate_up (K 4096, N 28672) at M = 2048 leaves 3.5 rounds of 256 x 256 tiles on 256 CUs, and
    qkv (N 6144) at M = 4096 1.5 rounds; the tiled GEMM then runs the full rounds and re-tiles the
    last columns (128 x 256) in a second launch. Every output still sums K in increasing order, so
    the M rows equal, bit for bit, the same rows computed at M + 1, whose block rows do not
    split."""
    k = 4096
    gen = torch.Generator(device="cpu").manual_seed(4242)
    w = (torch.randn(n, k, generator=gen) * 0.02).to(dev)
    q, s = pkg.ops.quantize_weight_per_channel(w)
    del w
    x = torch.randn(m + 1, k, generator=gen).to(torch.bfloat16).to(dev)
    if mode == "glu":
        qp = pkg.ops.pack_glu(q)
        run = lambda xx: pkg.ops.w8a16_glu(xx, qp, s, algo=PREFILL)  # noqa: E731
    elif mode == "w8a8":
        qp = pkg.ops.pack_weight(q)
        run = lambda xx: pkg.ops.w8a8_linear(xx, qp, s)  # noqa: E731
    else:
        qp = pkg.ops.pack_weight(q)
        run = lambda xx: pkg.ops.w8a16_linear(xx, qp, s, algo=PREFILL)  # noqa: E731
    a, b = run(x[:m]), run(x)
    assert torch.equal(a.view(torch.int16), b[:m].view(torch.int16))


def _abi_prefill(pkg, dev, x, qp, s, n, ldy):
    """The tiled GEMM through the C ABI into an (M, ldy) buffer; the columns past n must stay
    untouched."""
    m, k = x.shape
    out = torch.full((m, ldy), -7.0, dtype=torch.bfloat16, device=dev)
    ws = pkg.ops.workspace(0, m, n, k, dev)
    status = pkg.library().lse_w8a16_gemm_algo(
        x.data_ptr(), k, qp.data_ptr(), s.data_ptr(), out.data_ptr(), ldy, m, n, k, PREFILL,
        ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0,
        torch.cuda.current_stream().cuda_stream)
    assert status == 0
    torch.cuda.synchronize()
    assert torch.all(out[:, n:] == -7.0), "kernel wrote outside y's rows"
    return out[:, :n]


@pytest.mark.parametrize("m,n,k", [(2048, 28672, 4096), (8192, 6144, 4096), (8000, 6140, 1024)])
def test_staged_output_tiles_bit_identical(pkg, dev, m, n, k):
    """W8A16 256 x 256 launches of three or more rounds of blocks on 256 CUs (gate_up at 2048
    tokens: 768 blocks in its full rounds; 6144 rows at 8192: 768; 8000 x 6140: 768, the last
    block row 64 tokens, the last block column 252 rows, a partial 16-byte chunk) stage each
    output tile through LDS when y's rows are 16-byte aligned (row stride a multiple of 8) and
    store it directly otherwise. Both give the same bits; the ragged case also against the fp64
    product on the GPU."""
    gen = torch.Generator(device="cpu").manual_seed(5150 + m + n)
    w = (torch.randn(n, k, generator=gen) * 0.02).to(dev)
    q, s = pkg.ops.quantize_weight_per_channel(w)
    del w
    qp = pkg.ops.pack_weight(q)
    x = torch.randn(m, k, generator=gen).to(torch.bfloat16).to(dev)
    ld_staged = (n + 8) // 8 * 8
    ld_direct = ld_staged + 4
    a = _abi_prefill(pkg, dev, x, qp, s, n, ld_staged)
    b = _abi_prefill(pkg, dev, x, qp, s, n, ld_direct)
    assert torch.equal(a.contiguous().view(torch.int16), b.contiguous().view(torch.int16))
    if n % 8:
        golden = (x.double() @ q.double().t()) * s.double()[None, :]
        ok, msg = check_rows_in_chunks(a.contiguous(), golden)
        assert ok, f"M={m} N={n}: {msg}"


@pytest.mark.parametrize("k", [64, 80, 1040])
def test_ping_pong_tile_with_short_and_odd_k(pkg, dev, k):
    """The W8A16 256 x 256 tile runs two wave rows half a stage apart over groups of three stage
    slots: one K step (64), two with a 16-wide tail (80) and 17 steps (1040) leave the last group
    partly empty. On 256 CUs 3000 x 20000 runs that tile over its first 16384 rows (768 blocks in
    three rounds, the last block row 184 tokens) and 256 x 192 tiles over the rest; staged output
    with a 16-byte aligned row stride, direct stores without: the same bits, within the tolerance
    of the fp64 product on the GPU, and row for row the bits of the first 1100 rows run alone
    (128 x 256 tiles, same summation order)."""
    m, n = 3000, 20000
    gen = torch.Generator(device="cpu").manual_seed(6100 + k)
    w = (torch.randn(n, k, generator=gen) * 0.02).to(dev)
    q, s = pkg.ops.quantize_weight_per_channel(w)
    del w
    qp = pkg.ops.pack_weight(q)
    x = torch.randn(m, k, generator=gen).to(torch.bfloat16).to(dev)
    a = _abi_prefill(pkg, dev, x, qp, s, n, n)
    b = _abi_prefill(pkg, dev, x, qp, s, n, n + 4)
    assert torch.equal(a.contiguous().view(torch.int16), b.contiguous().view(torch.int16)), f"K={k}"
    golden = (x.double() @ q.double().t()) * s.double()[None, :]
    ok, msg = check_rows_in_chunks(a.contiguous(), golden)
    assert ok, f"K={k}: {msg}"
    del golden
    y_small = pkg.ops.w8a16_linear(x[:1100], qp, s, algo=PREFILL)
    assert torch.equal(a[:1100].contiguous().view(torch.int16), y_small.view(torch.int16)), f"K={k}"
