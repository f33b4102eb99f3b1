"""Fused gate/up + SiLU-mul on the GPU (LlamaMLP's `act_fn(gate_proj(x)) * up_proj(x)`,
transformers modeling_llama.py:175), through the C ABI, against the oracle on seeded inputs.

Tolerances:
* W8A16: the W8A16 rule (max-abs <= 1e-2 * max|golden|, rel <= 1e-2 where |golden| >
  1e-3 * max|golden|), golden in fp64 over the same int8 weights.
* W8A8: g and u are exact functions of the int32 sums, so the only error is the fp32 SiLU and
  product before one bf16 rounding: every output within 1 bf16 ulp of the fp64 golden.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bf16_bits, to_bf16_tensor
from oracle import numerics as ora

pytestmark = pytest.mark.gpu

AUTO, DECODE, PREFILL = 0, 1, 2


def _inputs(seed, m, i, k, outliers=False):
    x_bits, w = ora.seeded_inputs(seed, m, 2 * i, k, outliers)
    q, s = ora.quantize_weight_per_channel(w)  # stacked [gate; up]
    return x_bits, q, s


def _device_weights(pkg, dev, q, s):
    return pkg.ops.pack_glu(torch.from_numpy(q).to(dev)), torch.from_numpy(s).to(dev)


def _w8a16(pkg, dev, x_bits, q, s, algo):
    qp, st = _device_weights(pkg, dev, q, s)
    h = pkg.ops.w8a16_glu(to_bf16_tensor(x_bits, dev), qp, st, algo=algo)
    torch.cuda.synchronize()
    return bf16_bits(h)


def _check_w8a16(pkg, dev, m, i, k, seed, algo):
    x_bits, q, s = _inputs(seed, m, i, k)
    h = _w8a16(pkg, dev, x_bits, q, s, algo)
    assert h.shape == (m, i)
    ok, msg = ora.within_tolerance(h, ora.w8a16_glu_golden(x_bits, q, s))
    assert ok, f"M={m} I={i} K={k} algo={algo}: {msg}"
    return x_bits, q, s, h


def _check_w8a8(pkg, dev, m, i, k, seed):
    x_bits, q, s = _inputs(seed, m, i, k, outliers=True)
    qp, st = _device_weights(pkg, dev, q, s)
    x = to_bf16_tensor(x_bits, dev)
    h = bf16_bits(pkg.ops.w8a8_glu(x, qp, st))
    xq, sx = ora.quantize_act_per_token(x_bits)
    golden = ora.w8a8_glu_golden(ora.w8a8_accumulate(xq, q), sx, s)
    ulps = ora.bf16_ulps_apart(h, golden)
    worst = np.unravel_index(np.argmax(ulps), ulps.shape) if ulps.size else None
    assert ulps.size == 0 or ulps.max() <= 1.0, (
        f"M={m} I={i} K={k}: {ulps.max():.2f} ulps at {worst}")


def test_pack_glu_bit_exact(pkg, dev):
    """The GPU packer against the oracle's layout, with padding past I and K, and the inverse."""
    rng = np.random.default_rng(5)
    for i, k in ((1, 16), (20, 80), (200, 1040), (14336, 4096)):
        q = rng.integers(-127, 128, (2 * i, k)).astype(np.int8)
        qp = pkg.ops.pack_glu(torch.from_numpy(q).to(dev))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(qp.cpu().numpy(), ora.pack_glu(q), err_msg=f"{i}x{k}")
        np.testing.assert_array_equal(pkg.ops.unpack_glu(qp, i, k).cpu().numpy(), q)
        assert qp.numel() == pkg.library().lse_packed_glu_bytes(i, k)


@pytest.mark.parametrize("m", [1, 2, 8, 15, 16, 17, 31, 32, 33, 48, 64])
def test_decode_all_m_tiles(pkg, dev, m):
    _check_w8a16(pkg, dev, m, 200, 1024, 200 + m, DECODE)


@pytest.mark.parametrize("m", [1, 16, 17, 33, 64])
@pytest.mark.parametrize("i,k", [(8, 16), (24, 80), (1000, 1040), (64, 8208), (3000, 256)])
def test_decode_ragged_shapes(pkg, dev, m, i, k):
    """I not a multiple of 16 (partial last tile pair), K tails, a deep K with few panels, and
    (M <= 16) activations both staged whole and streamed."""
    _check_w8a16(pkg, dev, m, i, k, 13 * m + i + k, DECODE)


@pytest.mark.parametrize("m", [1, 17, 65, 128, 129, 300])
@pytest.mark.parametrize("i,k", [(64, 64), (100, 112), (200, 1040), (520, 2048)])
def test_prefill_ragged_shapes(pkg, dev, m, i, k):
    _check_w8a16(pkg, dev, m, i, k, 5 * m + i + k, PREFILL)


@pytest.mark.parametrize("m", [1, 32, 64, 65, 512])
def test_llama_gate_up_full_size(pkg, dev, m):
    """Llama-3-8B's gate/up: I = 14336, K = 4096 (the fused N = 28672 of the benchmarks)."""
    _check_w8a16(pkg, dev, m, 14336, 4096, 1000 + m, AUTO)


@pytest.mark.parametrize("algo", [DECODE, PREFILL])
def test_decode_and_prefill_agree_with_the_unfused_chain(pkg, dev, algo):
    """The fused result against the unfused path it replaces: the stacked W8A16 GEMM (bf16 g
    and u), then SiLU and the product in bf16, as the reference's LlamaMLP rounds them. They
    differ by the three extra roundings only: at most a few bf16 ulps, and the fused result is
    the closer one to the fp64 golden on average."""
    m, i, k = (24 if algo == DECODE else 160), 520, 2048
    x_bits, q, s = _inputs(77, m, i, k)
    h = _w8a16(pkg, dev, x_bits, q, s, algo)
    x = to_bf16_tensor(x_bits, dev)
    qp = pkg.ops.pack_weight(torch.from_numpy(q).to(dev))
    gu = pkg.ops.w8a16_linear(x, qp, torch.from_numpy(s).to(dev), algo=algo)
    chain = bf16_bits(torch.nn.functional.silu(gu[:, :i]) * gu[:, i:])
    golden = ora.w8a16_glu_golden(x_bits, q, s)
    gmax = np.abs(golden).max()
    big = np.abs(golden) > 1e-2 * gmax
    fused_ulps = ora.bf16_ulps_apart(h, golden)[big]
    chain_ulps = ora.bf16_ulps_apart(chain, golden)[big]
    assert fused_ulps.max() <= 2.0, fused_ulps.max()
    assert chain_ulps.max() <= 6.0, chain_ulps.max()
    assert fused_ulps.mean() < chain_ulps.mean(), (fused_ulps.mean(), chain_ulps.mean())


@pytest.mark.parametrize("m", [1, 16, 17, 33, 64, 65, 300])
@pytest.mark.parametrize("i,k", [(200, 1024), (24, 80)])
def test_w8a8_within_one_ulp(pkg, dev, m, i, k):
    _check_w8a8(pkg, dev, m, i, k, 3 * m + i)


def test_w8a8_llama_gate_up_full_size(pkg, dev):
    for m in (1, 64, 100, 512):
        _check_w8a8(pkg, dev, m, 14336, 4096, 50 + m)


def test_silu_tails(pkg, dev):
    """Unit activations and scale 1 make g and u small integers: g = -100 (e^100 overflows, silu
    -> -0), g = 0 (-> 0), g = +100 (-> 100), times u exactly."""
    i, k = 16, 64
    q = np.zeros((2 * i, k), np.int8)
    q[0, 0], q[1, 1], q[2, 2] = -100, 0, 100
    q[i + 0, 0], q[i + 1, 1], q[i + 2, 2] = 3, 5, 7
    q[3, 3], q[i + 3, 3] = 1, 1
    s = np.ones(2 * i, np.float32)
    x = np.zeros((1, k), np.float32)
    x[0, :4] = 1.0
    x_bits = ora.f32_to_bf16_bits(x)
    for algo in (DECODE, PREFILL):
        h = ora.bf16_bits_to_f32(_w8a16(pkg, dev, x_bits, q, s, algo))[0]
        assert h[0] == 0.0 and np.signbit(h[0]), h[0]
        assert h[1] == 0.0 and h[2] == 700.0, h[:3]
        assert h[3] == ora.bf16_bits_to_f32(ora.f64_to_bf16_bits(np.array([ora.silu64(1.0)])))[0]
        assert np.all(h[4:] == 0.0)


@pytest.mark.parametrize("algo", [DECODE, PREFILL])
def test_output_stride_guard_band(pkg, dev, algo):
    """h with a row stride past I: the kernels write exactly the I columns of each row."""
    m, i, k = 20, 40, 256
    x_bits, q, s = _inputs(8, m, i, k)
    qp, st = _device_weights(pkg, dev, q, s)
    x = to_bf16_tensor(x_bits, dev)
    pad = 9
    out = torch.full((m, i + pad), -7.0, dtype=torch.bfloat16, device=dev)
    status = pkg.library().lse_w8a16_glu(
        x.data_ptr(), k, qp.data_ptr(), st.data_ptr(), out.data_ptr(), i + pad, m, i, k, algo,
        torch.cuda.current_stream().cuda_stream)
    assert status == 0
    torch.cuda.synchronize()
    assert torch.all(out[:, i:] == -7.0)
    ok, msg = ora.within_tolerance(bf16_bits(out[:, :i]), ora.w8a16_glu_golden(x_bits, q, s))
    assert ok, msg


@pytest.mark.parametrize("i,k", [(300, 1024), (8200, 144)])
def test_decode_rows_are_batch_invariant(pkg, dev, i, k):
    """A row's result does not depend on the other rows of its token class, and every class
    meets the golden. I = 8200 (1026 packed row tiles) sends 17..64 tokens to the 32 x 128 and
    64 x 128 tiled routes."""
    x_bits, q, s = _inputs(31, 64, i, k)
    for lo, hi in ((1, 16), (17, 32), (33, 64)):
        full = _w8a16(pkg, dev, x_bits[:hi], q, s, DECODE)
        part = _w8a16(pkg, dev, x_bits[:lo], q, s, DECODE)
        np.testing.assert_array_equal(part, full[:lo], err_msg=f"class {lo}..{hi}")
        ok, msg = ora.within_tolerance(full, ora.w8a16_glu_golden(x_bits[:hi], q, s))
        assert ok, f"I={i} K={k} M={hi}: {msg}"


def test_rejections(pkg, dev):
    lib = pkg.library()
    stream = torch.cuda.current_stream().cuda_stream
    qp = torch.zeros(pkg.ops.packed_glu_shape(16, 64), dtype=torch.int8, device=dev)
    s = torch.ones(32, dtype=torch.float32, device=dev)
    x = torch.zeros(4, 64, dtype=torch.bfloat16, device=dev)
    h = torch.zeros(4, 16, dtype=torch.bfloat16, device=dev)
    args = (x.data_ptr(), 64, qp.data_ptr(), s.data_ptr(), h.data_ptr(), 16)
    assert lib.lse_w8a16_glu(*args, 4, 16, 40, AUTO, stream) == -3     # K % 16
    assert lib.lse_w8a16_glu(*args, 4, -1, 64, AUTO, stream) == -2     # negative I
    assert lib.lse_w8a16_glu(*args, 65, 16, 64, DECODE, stream) == -5  # decode past 64 rows
    assert lib.lse_w8a16_glu(x.data_ptr(), 64, qp.data_ptr(), s.data_ptr(), h.data_ptr(), 8, 4,
                             16, 64, AUTO, stream) == -2               # ldh < I
    assert lib.lse_w8a8_glu(None, None, qp.data_ptr(), s.data_ptr(), h.data_ptr(), 16, 4, 16, 64,
                            stream) == -1
    with pytest.raises(RuntimeError, match="gate/up scales"):
        pkg.ops.w8a16_glu(x, qp, s[:31])
    with pytest.raises(RuntimeError, match="packed weight"):
        pkg.ops.w8a16_glu(x, qp, torch.ones(34, dtype=torch.float32, device=dev))


def test_gate_up_module_and_mlp_drop_in(pkg, dev):
    """Int8GluMLP computes LlamaMLP.forward, down_proj(act_fn(gate_proj(x)) * up_proj(x)), as
    down_proj(gate_up(x)); gate_up meets the oracle, the whole stays within quantization error of
    the bf16 LlamaMLP, and a graph replays it bit-identically."""
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaMLP

    torch.manual_seed(0)
    cfg = LlamaConfig(hidden_size=256, intermediate_size=688, hidden_act="silu")
    mlp = LlamaMLP(cfg).to(device=dev, dtype=torch.bfloat16)
    for lin in (mlp.gate_proj, mlp.up_proj, mlp.down_proj):
        torch.nn.init.normal_(lin.weight, std=0.02)
    for mode in ("int8", "w8a8"):
        fused = pkg.Int8GluMLP.from_mlp(mlp, mode)
        gu = fused.gate_up
        q = gu.unpacked_qweight().cpu().numpy()
        s = gu.scales.cpu().numpy()
        q_ref, s_ref = ora.quantize_weight_per_channel(
            torch.cat([mlp.gate_proj.weight, mlp.up_proj.weight]).detach().float().cpu().numpy())
        np.testing.assert_array_equal(q, q_ref)
        np.testing.assert_array_equal(s, s_ref)
        x = torch.randn(3, 9, 256, device=dev).to(torch.bfloat16)
        y = fused(x)
        assert y.shape == (3, 9, 256) and y.dtype == torch.bfloat16
        h = gu(x)
        assert torch.equal(y, fused.down_proj(h))
        x_bits, h_bits = bf16_bits(x.reshape(-1, 256)), bf16_bits(h.reshape(-1, 688))
        if mode == "int8":
            ok, msg = ora.within_tolerance(h_bits, ora.w8a16_glu_golden(x_bits, q, s))
            assert ok, msg
        else:
            xq, sx = ora.quantize_act_per_token(x_bits)
            golden = ora.w8a8_glu_golden(ora.w8a8_accumulate(xq, q), sx, s)
            assert ora.bf16_ulps_apart(h_bits, golden).max() <= 1.0
        with torch.no_grad():
            ref = mlp(x).float()
        err = (y.float() - ref).abs().max().item()
        assert err <= 0.05 * ref.abs().max().item(), (mode, err)
        static_x = torch.randn(16, 256, device=dev).to(torch.bfloat16)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fused(static_x)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            static_y = fused(static_x)
        for rep in range(3):
            static_x.copy_(torch.randn(16, 256, device=dev).to(torch.bfloat16))
            graph.replay()
            torch.cuda.synchronize()
            eager = fused(static_x)
            torch.cuda.synchronize()
            assert torch.equal(static_y, eager), f"replay {rep} ({mode})"


def test_quantize_model_fuses_the_mlp(pkg, dev):
    """quantize_model_ swaps each LlamaMLP for Int8GluMLP; logits stay close to bf16's and to
    the unfused int8 model's."""
    from transformers import LlamaConfig, LlamaForCausalLM

    config = LlamaConfig(
        vocab_size=64, hidden_size=64, intermediate_size=176, num_hidden_layers=2,
        num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64,
        bos_token_id=None, eos_token_id=None, pad_token_id=None,
    )
    ids = torch.randint(0, 64, (1, 12), device=dev)
    logits = {}
    for fuse in (None, True, False):
        torch.manual_seed(0)
        model = LlamaForCausalLM(config).to(device=dev, dtype=torch.bfloat16).eval()
        if fuse is not None:
            pkg.quantize_model_(model, "int8", fuse_mlp=fuse)
            for layer in model.model.layers:
                assert isinstance(layer.mlp, pkg.Int8GluMLP) == fuse
        with torch.no_grad():
            logits[fuse] = model(ids).logits.float()
    scale = logits[None].abs().max().item()
    assert (logits[True] - logits[None]).abs().max().item() <= 0.05 * scale
    assert (logits[True] - logits[False]).abs().max().item() <= 0.02 * scale


def test_w8a16_96_row_tiles(pkg, dev):
    """Fused gate/up at 65..96 tokens in one block row of 96 x 128 tiles (I 8500: 133 blocks of
    64 gate/up row pairs, the last partly past I): against the oracle at 80 tokens, and row for
    row the same bits as inside 100 tokens (128 x 128 tiles)."""
    i, k = 8500, 1024
    x_bits, q, s = _inputs(9601, 100, i, k)
    qp, st = _device_weights(pkg, dev, q, s)
    x = to_bf16_tensor(x_bits, dev)
    h100 = bf16_bits(pkg.ops.w8a16_glu(x, qp, st, algo=PREFILL))
    h80 = bf16_bits(pkg.ops.w8a16_glu(x[:80], qp, st, algo=PREFILL))
    ok, msg = ora.within_tolerance(h80, ora.w8a16_glu_golden(x_bits[:80], q, s))
    assert ok, msg
    np.testing.assert_array_equal(h80, h100[:80])
